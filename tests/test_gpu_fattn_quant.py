"""GPU parity of FlashAttention decode over a quantized KV cache (q8_0 / q4_0 K and V, dequantized in-kernel).

The reference semantics are attention over the dequantized cache, d * q per element (ggml's dequantize_q8_0 /
dequantize_q4_0, exact in FP32): the oracle's attention_reference runs on those exact values, and the kernel is
held to the same bar as the fp16 path (include/p100/tolerance.h element-wise, max relative 2e-3). Shapes: the
decode configuration, d 64 / 256 with GQA ratios, several query rows with causal alignment and masks, softcap, a
ggml-style interleaved cache view, and the device-side KV length.
"""
import numpy as np
import pytest

import p100_amd as P

from test_gpu_fattn import to_dev
from test_gpu_decode import deq_rows

pytestmark = pytest.mark.gpu


def quant(kv_type, x):
    """x float32 [rows, d] -> (GGUF blocks uint8 [rows, d/32 * block bytes], exact dequantized float32 [rows, d])."""
    import torch

    from p100_amd import synth

    t = P.TYPES[kv_type]
    blocks = synth.QUANTIZERS[t](torch.from_numpy(np.ascontiguousarray(x, np.float32))).numpy()
    return blocks, deq_rows(t, blocks)


def poison_rows(blocks, p, first, d):
    """Rows at positions >= first of every (batch, KV head) get a NaN / Inf fp16 scale in every block and random
    quants (rows past the visible length are not valid; their bytes are arbitrary)."""
    rb = blocks.shape[1]
    b = blocks.reshape(p.batch, p.n_head_kv, p.seq_kv, rb).copy()
    bb = rb // (d // 32)
    tail = b[:, :, first:]
    tail[...] = np.random.default_rng(first).integers(0, 256, tail.shape, dtype=np.uint8)
    for blk in range(d // 32):
        bits = np.uint16(0x7E00 if blk % 2 == 0 else 0x7C00)  # NaN, +Inf
        tail[..., blk * bb] = bits & 255
        tail[..., blk * bb + 1] = bits >> 8
    return b.reshape(-1, rb)


def run(orc, kv_type, p, seed=0, mask=None, scale_kv=1.0, strided=False, kv_len=None, check_len=None,
        poison=False):
    rng = np.random.default_rng(seed)
    nq = p.batch * p.n_head_q * p.seq_q * p.d_qk
    rows = p.batch * p.n_head_kv * p.seq_kv
    q = rng.standard_normal(nq).astype(np.float32)
    kb, kd = quant(kv_type, (rng.standard_normal((rows, p.d_qk)) * scale_kv).astype(np.float32))
    vb, vd = quant(kv_type, (rng.standard_normal((rows, p.d_v)) * scale_kv).astype(np.float32))
    dp = P.AttnParams(p.batch, p.n_head_q, p.n_head_kv, p.seq_q, p.seq_kv, p.d_qk, p.d_v, p.scale, p.softcap,
                      bool(p.causal))
    strides = None
    if poison:  # only the first kv_len rows are read as valid; the reference sees the unpoisoned ones
        kb, vb = poison_rows(kb, p, kv_len, p.d_qk), poison_rows(vb, p, kv_len, p.d_v)
    kdev, vdev = to_dev(kb), to_dev(vb)
    if strided:  # ggml's cache view: rows of all KV heads interleaved per position ([batch][seq_kv][head][row])
        rb = kb.shape[1]
        perm = lambda a: a.reshape(p.batch, p.n_head_kv, p.seq_kv, rb).transpose(0, 2, 1, 3).copy()
        kdev, vdev = to_dev(perm(kb)), to_dev(perm(vb))
        strides = P.KVStrides(p.n_head_kv * rb, rb, p.seq_kv * p.n_head_kv * rb,
                              p.n_head_kv * rb, rb, p.seq_kv * p.n_head_kv * rb)
    lend = None if kv_len is None else to_dev(np.int32([kv_len]))
    o, lse = P.flash_attn_decode_quant(dp, kv_type, to_dev(q), kdev, vdev,
                                       mask=None if mask is None else to_dev(mask), byte_strides=strides, kv_len=lend)
    pr = p
    kref, vref = kd, vd
    if check_len is not None:  # the reference over the first check_len positions
        pr = orc.AttnParams(p.batch, p.n_head_q, p.n_head_kv, p.seq_q, check_len, p.d_qk, p.d_v, p.scale, p.softcap,
                            bool(p.causal))
        kref = kd.reshape(p.batch, p.n_head_kv, p.seq_kv, -1)[:, :, :check_len]
        vref = vd.reshape(p.batch, p.n_head_kv, p.seq_kv, -1)[:, :, :check_len]
    ref, ref_lse = orc.attention_reference(pr, q, kref, vref, mask)
    o, lse = o.cpu().numpy(), lse.cpu().numpy()
    r = ref.astype(np.float64)
    err = np.abs(o.astype(np.float64) - r)
    assert np.isfinite(o).all()
    assert not (err > 1e-3 + 2e-3 * np.abs(r)).any(), err.max()
    assert err.max() / max(np.abs(r).max(), 1e-30) <= 2e-3
    neg = np.isneginf(ref_lse)
    assert (np.isneginf(lse) == neg).all()
    r_l = ref_lse[~neg].astype(np.float64)
    assert (np.abs(lse[~neg].astype(np.float64) - r_l) <= 1e-3 + 4 * 2.0 ** -23 * np.abs(r_l)).all()


KV_TYPES = ["q8_0", "q4_0"]


@pytest.mark.parametrize("kv_type", KV_TYPES)
@pytest.mark.parametrize("seq_kv", [1, 7, 64, 1000, 8192])
@pytest.mark.parametrize("causal", [False, True])
def test_decode_config(orc, gpu, kv_type, seq_kv, causal):
    run(orc, kv_type, orc.AttnParams(1, 32, 8, 1, seq_kv, 128, 128, 0.0, 0.0, causal), seed=seq_kv)


@pytest.mark.parametrize("kv_type", KV_TYPES)
@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("group", [1, 4])
def test_shapes(orc, gpu, kv_type, d, group):
    run(orc, kv_type, orc.AttnParams(2, 2 * group, 2, 1, 65, d, d, 0.0, 0.0, False), seed=d + group)


@pytest.mark.parametrize("kv_type", KV_TYPES)
def test_rows_mask_softcap(orc, gpu, kv_type):
    p = orc.AttnParams(1, 8, 2, 3, 200, 128, 128, 0.0, 0.0, True)
    run(orc, kv_type, p, seed=5)
    mask = np.zeros((3, 200), np.float32)
    mask[0, :] = -np.inf  # a fully masked row: o = 0, lse = -inf
    mask[1, 50:120] = -np.inf
    mask[2, ::3] = -1.5
    run(orc, kv_type, orc.AttnParams(1, 8, 2, 3, 200, 128, 128, 0.0, 0.0, False), seed=6, mask=mask)
    run(orc, kv_type, orc.AttnParams(1, 8, 2, 1, 300, 128, 128, 0.0, 20.0, False), seed=7, scale_kv=4.0)


@pytest.mark.parametrize("kv_type", KV_TYPES)
def test_strided_cache_view_and_device_length(orc, gpu, kv_type):
    run(orc, kv_type, orc.AttnParams(1, 32, 8, 1, 777, 128, 128, 0.0, 0.0, False), seed=8, strided=True)
    for n in (1, 513, 1024):
        run(orc, kv_type, orc.AttnParams(1, 32, 8, 1, 1024, 128, 128, 0.0, 0.0, False), seed=9, kv_len=n,
            check_len=n)


@pytest.mark.parametrize("kv_type", KV_TYPES)
@pytest.mark.parametrize("n", [1, 63, 513, 1000])
def test_rows_past_device_length_may_hold_nan(orc, gpu, kv_type, n):
    """NaN / Inf block scales and random quants in the rows past the device-side length never reach O or LSE."""
    run(orc, kv_type, orc.AttnParams(1, 32, 8, 1, 1024, 128, 128, 0.0, 0.0, False), seed=10 + n, kv_len=n,
        check_len=n, poison=True)


def test_random_shapes(orc, gpu):
    """A fixed-seed sweep of 24 cases: q8_0 or q4_0, batch 1..2, KV heads 1..8 with GQA ratios 1..8, d 64 / 128 /
    256, 1..4 query rows, 1..3000 keys, causal or not, a mask or none, softcap or none, the dense layout or the
    interleaved cache view, and (unmasked, non-causal) a device-side length with poisoned rows past it."""
    g = np.random.default_rng(4343)
    for case in range(24):
        kv_type = str(g.choice(KV_TYPES))
        hkv = int(g.integers(1, 9))
        seq_q, seq_kv = int(g.integers(1, 5)), int(g.integers(1, 3001))
        d = int(g.choice([64, 128, 256]))
        causal = bool(g.integers(0, 2))
        softcap = float(g.choice([0.0, 0.0, 4.0]))
        p = orc.AttnParams(int(g.integers(1, 3)), hkv * int(g.integers(1, 9)), hkv, seq_q, seq_kv, d, d,
                           float(g.choice([0.0, 0.0, 0.3])), softcap, causal)
        mask, strided, kv_len = None, bool(g.integers(0, 2)), None
        if g.integers(0, 2):
            mask = (0.5 * g.standard_normal((seq_q, seq_kv))).astype(np.float32)
            mask[g.random(mask.shape) < 0.2] = -np.inf
        elif not causal and not strided and g.integers(0, 2):
            kv_len = int(g.integers(1, seq_kv + 1))
        print(f"case {case}: {kv_type} b {p.batch} hq {p.n_head_q} hkv {hkv} sq {seq_q} skv {seq_kv} d {d} "
              f"causal {causal} mask {mask is not None} softcap {softcap} scale {p.scale} strided {strided} "
              f"kv_len {kv_len}", flush=True)
        run(orc, kv_type, p, seed=6000 + case, mask=mask, strided=strided, kv_len=kv_len, check_len=kv_len,
            poison=kv_len is not None)


def test_rejects_bad_arguments(gpu):
    import torch

    p = P.AttnParams(1, 4, 2, 1, 16, 128, 128)
    q = torch.zeros(4 * 128, device="cuda")
    k = torch.zeros(2 * 16 * 136 + 8, dtype=torch.uint8, device="cuda")
    with pytest.raises(P.P1XError):
        P.flash_attn_decode_quant(p, "q4_K", q, k, k)
    with pytest.raises(ValueError, match="4-byte aligned"):
        P.flash_attn_decode_quant(p, "q8_0", q, k[2:], k)
    bad = P.KVStrides(138, 138 * 16, 0, 136, 136 * 16, 0)
    with pytest.raises(ValueError, match="4-byte aligned"):
        P.flash_attn_decode_quant(p, "q8_0", q, k, k, byte_strides=bad)
