"""GPU parity of the split-K FlashAttention decode against the FP64 oracle (p100::attention_reference).

Bar: include/p100/tolerance.h:20-31 element-wise (|o-ref| <= 1e-3 + 2e-3|ref|, LSE within 1e-3, -inf exact),
and the path's stated "max relative error <= 2e-3" read as max|o-ref| / max|ref| (tests/error_budget.cpp:78).
Inputs are rounded to fp16 (the kernel's K/V type) on the host; Q stays fp32. Shapes: the decode config
(32 query heads / 8 KV heads, d 128, 1 query row, KV 512..32768, causal), plus GQA ratios 1..8, d 64 / 256,
batch 2, several query rows with bottom-right causal alignment, masks with fully masked rows, softcap,
large logits, the error-budget distributions (outlier channels, peaked, biased V), strided K/V views and a
fixed-seed sweep of random shapes.
The reference's analytic cases (tests/test_reference.cpp) run on the GPU with q/k/v zero-padded to d = 64,
which leaves every dot product and the first d_v output columns unchanged.
"""
import math

import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("fa_kernel")]

INF = math.inf


def to_dev(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def gen(orc, p, seed, dist="normal"):
    rng = np.random.default_rng(seed)
    nq, nk, nv, _, _ = p.shapes()
    q = rng.standard_normal(nq).astype(np.float32)
    k = rng.standard_normal(nk).astype(np.float32)
    v = rng.standard_normal(nv).astype(np.float32)
    if dist == "outlier":
        q.reshape(-1, p.d_qk)[:, :4] *= 20
        k.reshape(-1, p.d_qk)[:, :4] *= 20
    if dist == "vbias":
        v.reshape(-1, p.d_v)[:, :8] += 2
    k16 = orc.round_to_fp16(k).astype(np.float16)
    v16 = orc.round_to_fp16(v).astype(np.float16)
    return q, k16, v16


def run_gpu(p, q, k16, v16, mask=None, strides=None, k_dev=None, v_dev=None):
    import p100_amd as P
    import torch

    kd = k_dev if k_dev is not None else to_dev(k16.view(np.int16)).view(torch.float16)
    vd = v_dev if v_dev is not None else to_dev(v16.view(np.int16)).view(torch.float16)
    o, lse = P.flash_attn_decode(p, to_dev(q), kd, vd, mask=None if mask is None else to_dev(mask),
                                 strides=strides)
    return o.cpu().numpy(), lse.cpu().numpy()


def check(orc, p, q, k16, v16, mask=None, **kw):
    o, lse = run_gpu(p, q, k16, v16, mask, **kw)
    ref, ref_lse = orc.attention_reference(p, q, k16.astype(np.float32), v16.astype(np.float32), mask)
    r = ref.astype(np.float64)
    err = np.abs(o.astype(np.float64) - r)
    assert np.isfinite(o).all()
    bad = err > 1e-3 + 2e-3 * np.abs(r)
    assert not bad.any(), (err.max(), np.argwhere(bad)[:4])
    neg = np.isneginf(ref_lse)
    assert (np.isneginf(lse) == neg).all()
    # tolerance.h's absolute 1e-3 on LSE, plus 4 float32 ulps of |LSE|: past |LSE| ~ 2048 the float spacing
    # itself exceeds 1e-3 (FP32 logits cannot resolve it; the reference's float output rounds the same way).
    r_l = ref_lse[~neg].astype(np.float64)
    assert (np.abs(lse[~neg].astype(np.float64) - r_l) <= 1e-3 + 4 * 2.0 ** -23 * np.abs(r_l)).all()
    max_rel = err.max() / max(np.abs(r).max(), 1e-30)
    assert max_rel <= 2e-3
    return max_rel


@pytest.mark.parametrize("seq_kv", [512, 2048, 8192])
@pytest.mark.parametrize("causal", [False, True])
def test_decode_config(orc, gpu, seq_kv, causal):
    p = orc.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=seq_kv, d_qk=128, d_v=128, causal=causal)
    q, k, v = gen(orc, p, seq_kv)
    rel = check(orc, p, q, k, v)
    print(f"seq_kv={seq_kv} causal={causal} max_rel={rel:.3e}")


def test_decode_32k(orc, gpu):
    p = orc.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=32768, d_qk=128, d_v=128, causal=True)
    q, k, v = gen(orc, p, 32768, "vbias")
    check(orc, p, q, k, v)


@pytest.mark.parametrize("dist", ["outlier", "vbias", "peaked"])
def test_error_budget_distributions(orc, gpu, dist):
    p = orc.AttnParams(n_head_q=8, n_head_kv=2, seq_q=1, seq_kv=4096, d_qk=128, d_v=128)
    if dist == "peaked":
        p.scale = 64.0 / math.sqrt(128)
    q, k, v = gen(orc, p, 12345, "normal" if dist == "peaked" else dist)
    check(orc, p, q, k, v)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("group", [1, 2, 3, 4, 8, 16])
def test_shapes(orc, gpu, d, group):
    for seq_kv in (1, 7, 65, 1000):
        p = orc.AttnParams(batch=2, n_head_q=2 * group, n_head_kv=2, seq_q=1, seq_kv=seq_kv, d_qk=d, d_v=d)
        q, k, v = gen(orc, p, seq_kv * d + group)
        check(orc, p, q, k, v)


def test_multi_row_causal_and_mask(orc, gpu):
    # seq_q > seq_kv: the first rows see no key (O = 0, LSE = -inf), as tests/test_reference.cpp:165-174.
    for sq, sk in ((5, 3), (3, 130), (16, 300)):
        p = orc.AttnParams(n_head_q=4, n_head_kv=2, seq_q=sq, seq_kv=sk, d_qk=128, d_v=128, causal=True)
        q, k, v = gen(orc, p, sq * sk)
        check(orc, p, q, k, v)
    p = orc.AttnParams(n_head_q=4, n_head_kv=1, seq_q=3, seq_kv=200, d_qk=64, d_v=64)
    q, k, v = gen(orc, p, 9)
    rng = np.random.default_rng(10)
    mask = rng.standard_normal((3, 200)).astype(np.float32)
    mask[0, :] = -INF               # a fully masked row
    mask[1, rng.random(200) < 0.7] = -INF
    check(orc, p, q, k, v, mask.ravel())


def test_random_shapes(orc, gpu):
    """A fixed-seed sweep of 32 cases: batch 1..2, KV heads 1..8 with GQA ratios 1..8, d 64 / 128 / 256, 1..4 query
    rows, 1..3000 keys (split plans from one split to many, partial last batches), causal or not, an additive mask
    with masked-out keys or none, softcap or none, the default or an explicit scale."""
    g = np.random.default_rng(777)
    for case in range(32):
        hkv = int(g.integers(1, 9))
        p = orc.AttnParams(batch=int(g.integers(1, 3)), n_head_q=hkv * int(g.integers(1, 9)), n_head_kv=hkv,
                           seq_q=int(g.integers(1, 5)), seq_kv=int(g.integers(1, 3001)),
                           d_qk=int(g.choice([64, 128, 256])), causal=bool(g.integers(0, 2)),
                           softcap=float(g.choice([0.0, 0.0, 4.0])), scale=float(g.choice([0.0, 0.0, 0.3])))
        p.d_v = p.d_qk
        mask = None
        if g.integers(0, 2):
            mask = (0.5 * g.standard_normal((p.seq_q, p.seq_kv))).astype(np.float32)
            mask[g.random(mask.shape) < 0.2] = -INF
            mask = mask.ravel()
        print(f"case {case}: b {p.batch} hq {p.n_head_q} hkv {hkv} sq {p.seq_q} skv {p.seq_kv} d {p.d_qk} "
              f"causal {p.causal} mask {mask is not None} softcap {p.softcap} scale {p.scale}", flush=True)
        q, k, v = gen(orc, p, 9000 + case)
        check(orc, p, q, k, v, mask)


def test_softcap_and_large_logits(orc, gpu):
    p = orc.AttnParams(n_head_q=8, n_head_kv=8, seq_q=1, seq_kv=777, d_qk=128, d_v=128, softcap=5.0, scale=0.5)
    q, k, v = gen(orc, p, 77)
    check(orc, p, q, k, v)
    p = orc.AttnParams(n_head_q=4, n_head_kv=4, seq_q=1, seq_kv=300, d_qk=64, d_v=64, scale=1000.0)
    q, k, v = gen(orc, p, 78)
    check(orc, p, q, k, v)


def test_workspace_reuse_and_graph_replay(orc, gpu):
    """One workspace serves a sequence of different calls and replays of a captured graph (two launches per
    call, the second reading the partials the first wrote), with eager calls between replays."""
    import p100_amd as P
    import torch

    cfgs = [orc.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=8192, d_qk=128, d_v=128, causal=True),
            orc.AttnParams(batch=2, n_head_q=6, n_head_kv=2, seq_q=3, seq_kv=300, d_qk=64, d_v=64, causal=True),
            orc.AttnParams(n_head_q=8, n_head_kv=8, seq_q=1, seq_kv=2000, d_qk=256, d_v=256)]
    need = max(P.flash_attn_decode_workspace(P._params(p)) for p in cfgs)
    ws = torch.full((need // 4 + 4,), float("nan"), dtype=torch.float32, device="cuda")  # contents arbitrary
    data = []
    for n, p in enumerate(cfgs):
        q, k, v = gen(orc, p, 500 + n)
        qd, kd, vd = to_dev(q), to_dev(k.view(np.int16)).view(torch.float16), to_dev(v.view(np.int16)).view(torch.float16)
        o = torch.empty(q.size, dtype=torch.float32, device="cuda")
        lse = torch.empty(p.batch * p.n_head_q * p.seq_q, dtype=torch.float32, device="cuda")
        data.append((P._params(p), qd, kd, vd, o, lse))
    eager = []
    for _ in range(2):  # each call twice, interleaved: results must not depend on what ran before
        for p, qd, kd, vd, o, lse in data:
            P.flash_attn_decode(p, qd, kd, vd, out=o, lse=lse, workspace=ws)
            eager.append((o.clone(), lse.clone()))
    for n in range(3):
        assert torch.equal(eager[n][0], eager[n + 3][0]) and torch.equal(eager[n][1], eager[n + 3][1])
    for (p, qd, kd, vd, o, lse), n in zip(data, range(3)):  # and they are right
        q = qd.cpu().numpy()
        ref, ref_lse = orc.attention_reference(cfgs[n], q, kd.cpu().numpy().astype(np.float32),
                                               vd.cpu().numpy().astype(np.float32))
        err = np.abs(eager[n][0].cpu().numpy().astype(np.float64) - ref)
        assert (err <= 1e-3 + 2e-3 * np.abs(ref)).all()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for p, qd, kd, vd, o, lse in data:
                P.flash_attn_decode(p, qd, kd, vd, out=o, lse=lse, workspace=ws, stream=side)
    for rep in range(3):
        for _, _, _, _, o, lse in data:
            o.fill_(float("nan"))
            lse.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for n, (_, _, _, _, o, lse) in enumerate(data):
            assert torch.equal(o, eager[n][0]) and torch.equal(lse, eager[n][1]), (rep, n)
        P.flash_attn_decode(data[1][0], *data[1][1:4], out=data[1][4], lse=data[1][5], workspace=ws)  # eager between
        torch.cuda.synchronize()


def test_strided_kv_view(orc, gpu):
    """K and V as views into a larger cache: [batch][head][capacity][d] with capacity > seq_kv, and a row pitch."""
    import p100_amd as P
    import torch

    p = orc.AttnParams(batch=2, n_head_q=8, n_head_kv=2, seq_q=1, seq_kv=500, d_qk=128, d_v=128, causal=True)
    q, k, v = gen(orc, p, 5)
    cap, pitch = 640, 136
    kc = np.zeros((2, 2, cap, pitch), np.float16)
    vc = np.zeros((2, 2, cap, pitch), np.float16)
    kc[:, :, :500, :128] = k.reshape(2, 2, 500, 128)
    vc[:, :, :500, :128] = v.reshape(2, 2, 500, 128)
    st = P.KVStrides(pitch, cap * pitch, 2 * cap * pitch, pitch, cap * pitch, 2 * cap * pitch)
    kd = to_dev(kc.view(np.int16)).view(torch.float16)
    vd = to_dev(vc.view(np.int16)).view(torch.float16)
    o, lse = run_gpu(p, q, k, v, strides=st, k_dev=kd, v_dev=vd)
    o2, lse2 = run_gpu(p, q, k, v)
    assert (o.view(np.uint32) == o2.view(np.uint32)).all() and (lse.view(np.uint32) == lse2.view(np.uint32)).all()


def _pad(a, rows, d_from, d_to):
    out = np.zeros((rows, d_to), np.float32)
    out[:, :d_from] = np.asarray(a, np.float32).reshape(rows, d_from)
    return out.ravel()


def reference_kat(orc, p, q, k, v, mask=None):
    """Runs an analytic case on the GPU with q/k/v zero-padded to d = 64; returns (o[:, :d_v], lse)."""
    D = 64
    # Padding d changes the default scale 1/sqrt(d_qk): pass the original effective scale explicitly.
    scale = p.scale if p.scale != 0.0 else float(np.float32(1) / np.sqrt(np.float32(p.d_qk)))
    pp = orc.AttnParams(p.batch, p.n_head_q, p.n_head_kv, p.seq_q, p.seq_kv, D, D, scale, p.softcap, bool(p.causal))
    nq = p.batch * p.n_head_q * p.seq_q
    nkv = p.batch * p.n_head_kv * p.seq_kv
    qd = _pad(q, nq, p.d_qk, D)
    kd = _pad(k, nkv, p.d_qk, D).astype(np.float16)
    vd = _pad(v, nkv, p.d_v, D).astype(np.float16)
    o, lse = run_gpu(pp, qd, kd, vd, None if mask is None else np.asarray(mask, np.float32))
    return o.reshape(nq, D)[:, :p.d_v].ravel(), lse


def test_reference_analytic_cases(orc, gpu):
    small = lambda nq, nk, dq, dv: orc.AttnParams(seq_q=nq, seq_kv=nk, d_qk=dq, d_v=dv, scale=1.0)
    ln3 = float(np.log(np.float32(3)))
    o, lse = reference_kat(orc, small(2, 2, 2, 2), [1, 0, 0, 1], [ln3, 0, 0, ln3], [2, 4, 6, 8])
    assert np.allclose(o, [3, 5, 5, 7], atol=2e-5) and np.allclose(lse, math.log(4), atol=2e-6)
    p = small(2, 3, 2, 3)
    p.scale = 0.0
    o, lse = reference_kat(orc, p, [0] * 4, [1, 2, 3, 4, 5, 6], [1, 2, 6, 3, 4, 0, 8, 9, -3])
    assert np.allclose(o.reshape(2, 3), [[4, 5, 1]] * 2, atol=1e-5) and np.allclose(lse, math.log(3), atol=2e-6)
    p = small(3, 5, 1, 1)
    p.causal = True
    o, lse = reference_kat(orc, p, [0, 0, 0], [0] * 5, [0, 2, 4, 6, 8])
    assert np.allclose(o, [2, 3, 4], atol=1e-5) and np.allclose(lse, np.log([3, 4, 5]), atol=2e-6)
    p.seq_q, p.seq_kv = 5, 3
    o, lse = reference_kat(orc, p, [0] * 5, [0] * 3, [0, 2, 4])
    assert list(o[:2]) == [0, 0] and np.isneginf(lse[:2]).all() and np.allclose(o[2:], [0, 1, 2], atol=1e-5)
    o, lse = reference_kat(orc, small(2, 3, 1, 2), [1, 1], [1, 2, 3], [1, 2, 3, 4, 5, 6],
                           [-INF, -INF, -INF, -INF, 0, -INF])
    assert list(o[:2]) == [0, 0] and lse[0] == -INF and np.allclose(o[2:], [3, 4]) and abs(lse[1] - 2) < 1e-6
    p = small(1, 2, 1, 1)
    p.scale, p.softcap = 2.0, 3.0
    o, lse = reference_kat(orc, p, [10], [10, -10], [2, 9], [-4, 1])
    a, b = 3 * math.tanh(200 / 3) - 4, 3 * math.tanh(-200 / 3) + 1
    s = math.exp(a) + math.exp(b)
    assert abs(o[0] - (2 * math.exp(a) + 9 * math.exp(b)) / s) <= 2e-5 and abs(lse[0] - math.log(s)) <= 1e-5
    p = small(1, 3, 1, 2)
    p.scale = 10000
    o, lse = reference_kat(orc, p, [1], [-1, 1, 0], [1, 2, 7, -3, 9, 10])
    assert list(o) == [7, -3] and lse[0] == 10000


def test_validation_reasons(orc, gpu):
    import p100_amd as P
    import torch

    z = torch.zeros(64, dtype=torch.float32, device="cuda")
    zh = torch.zeros(64, dtype=torch.float16, device="cuda")
    cases = [(dict(batch=0), "all dimensions must be positive"), (dict(d_v=-1), "all dimensions must be positive"),
             (dict(n_head_q=3, n_head_kv=2), "n_head_q must be divisible by n_head_kv"),
             (dict(softcap=-1.0), "softcap must be finite and non-negative"),
             (dict(softcap=INF), "softcap must be finite and non-negative"),
             (dict(scale=math.nan), "scale must be finite")]
    for kw, why in cases:
        p = P.AttnParams(**kw)
        assert P.validate(p) == why == orc.validate(orc.AttnParams(**kw))
        with pytest.raises(ValueError) as e:
            P.flash_attn_decode(p, z, zh, zh)
        assert str(e.value) == why
    with pytest.raises(P.P1XError):
        P.flash_attn_decode(P.AttnParams(d_qk=32, d_v=32), z, zh, zh)


@pytest.mark.parametrize("n", [1, 63, 513, 1000])
def test_rows_past_device_length_may_hold_nan(orc, gpu, n):
    """Rows in [kv_len, seq_kv) are not valid (their bits are arbitrary): filling them with fp16 NaN and Inf must
    not reach O or LSE. n leaves the last batch of a split partly past the visible end."""
    import p100_amd as P
    import torch

    cap, hq, hkv, d = 1024, 32, 8, 128
    rng = np.random.default_rng(n)
    q = rng.standard_normal(hq * d).astype(np.float32)
    k16 = rng.standard_normal((hkv, cap, d)).astype(np.float16)
    v16 = rng.standard_normal((hkv, cap, d)).astype(np.float16)
    kp, vp = k16.copy(), v16.copy()
    kp[:, n:, ::2] = np.float16(np.nan)
    kp[:, n:, 1::2] = np.float16(np.inf)
    vp[:, n:, ::2] = np.float16(-np.inf)
    vp[:, n:, 1::2] = np.float16(np.nan)
    p = P.AttnParams(1, hq, hkv, 1, cap, d, d, 0.0, 0.0, False)
    kd = to_dev(kp.view(np.int16)).view(torch.float16)
    vd = to_dev(vp.view(np.int16)).view(torch.float16)
    o, lse = P.flash_attn_decode(p, to_dev(q), kd, vd, kv_len=to_dev(np.int32([n])))
    o, lse = o.cpu().numpy(), lse.cpu().numpy()
    pm = orc.AttnParams(1, hq, hkv, 1, n, d, d, 0.0, 0.0, False)
    ref, ref_lse = orc.attention_reference(pm, q, k16[:, :n].astype(np.float32), v16[:, :n].astype(np.float32))
    assert np.isfinite(o).all() and np.isfinite(lse).all()
    err = np.abs(o.astype(np.float64) - ref)
    assert not (err > 1e-3 + 2e-3 * np.abs(ref)).any(), err.max()
    assert (np.abs(lse.astype(np.float64) - ref_lse) <= 1e-3).all()
