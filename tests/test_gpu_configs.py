"""GPU parity at the exact shapes of the benchmarked configurations, through the kernels those shapes dispatch.

The other GPU tests use small row counts (17 .. 3000 rows), which resolve to one row per wave; the benchmarked
matrices take other instantiations (two rows per wave for 4096 x 4096 in the single-launch form, two and four rows
per wave for the 14336- and 128256-row K-quant matrices, 64 threads per row in the h16 path, the register-resident
row-groups at 4096 .. 28672 rows). Each case here runs at full size through the public entry points:

* config 1: Q4_0 (and Q8_0) 4096 x 4096, one column, f32 activation (p1x_mul_mat_vec: one launch, Q8_1 in-kernel);
* config 2: the Llama-3-8B layer matrices (Wq/Wo 4096 x 4096, Wk/Wv 1024 x 4096, gate/up 14336 x 4096, down
  4096 x 14336), Q4_0 and Q8_0, ne11 in {1, 2, 4, 8}, through the f32 op and through a prepared Q8_1 activation;
* config 4: Q4_K 14336 x 4096 and 4096 x 14336, Q6_K 128256 x 4096 (and 4096 x 14336), one column;
* the h16 path at 4096 x 4096 and 14336 x 4096 for all four types;
* config 5: the 8B-shape decode step (32 layers) bit-identical to the same step composed from the separately
  tested entry points, after 600 positions; one 8B-dimension layer and the output head op by op against their
  references; and that layer end to end against the CPU restatement.

Bars (as tests/test_gpu_matvec.py): int32 group sums bit-exact; |y - oracle| <= 1e-5 * ||w_row|| * ||x||; never
further from FP64 than the oracle's own arithmetic (+1e-5); h16 within 1e-3 * ||w_row|| * ||x|| of FP64. Results
with and without the group-sum export are bit-identical (the export no longer changes the kernel shape).
Weights are N(0, 0.02) quantized on the GPU (p100_amd.synth), activations N(0, 1).
"""
from __future__ import annotations

import functools

import numpy as np
import pytest

import p100_amd as P

pytestmark = pytest.mark.gpu


def to_dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@functools.lru_cache(maxsize=4)
def weights(wtype, M, K, seed):
    """(device uint8 [M, row bytes], host copy) of N(0, 0.02) weights quantized on the GPU."""
    import torch

    from p100_amd import synth

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w = synth.random_weights(wtype, M, K, generator=g)
    return w, w.cpu().numpy()


def activation(K, ncols, seed):
    x = np.random.default_rng(seed).standard_normal((ncols, K)).astype(np.float32)
    x[:, :32] = 0  # one all-zero block (d = 0)
    x[:, 40] *= np.float32(50)  # an outlier
    return x


def check(orc, t, w, M, K, x, y, sums=None, mode="q81"):
    """y [ncols, M] (and the group sums) against the oracle; returns the worst model-relative error."""
    if mode == "q81":
        ref, ref_sums = orc.mul_mat_vec(t, w, M, K, x, want_sums=True)
    else:
        ref, ref_sums = orc.mul_mat_vec(t, w, M, K, x, mode=mode), None
    exact = orc.mul_mat_vec(t, w, M, K, x, mode="exact").astype(np.float64)
    scale = np.outer(np.linalg.norm(x.astype(np.float64), axis=1), orc.weight_norms(t, w, M, K))
    scale = np.where(scale > 0, scale, 1.0)
    if sums is not None:
        bad = np.argwhere(sums != ref_sums)
        assert bad.size == 0, f"{bad.shape[0]} group sums differ, first at [col, row, group] = {bad[0].tolist()}"
    assert np.isfinite(y).all()
    err = np.abs(y.astype(np.float64) - ref) / scale
    assert err.max() <= 1e-5, (err.max(), np.unravel_index(err.argmax(), err.shape))
    e_gpu = np.abs(y.astype(np.float64) - exact) / scale
    e_orc = np.abs(ref.astype(np.float64) - exact) / scale
    assert (e_gpu <= e_orc + 1e-5).all()
    if mode != "q81":
        assert e_gpu.max() <= 1e-3, e_gpu.max()
    return float(err.max())


def run_op(t, wd, M, K, x, with_sums=True):
    """The f32 op (p1x_mul_mat_vec) with and without the group-sum export; both must agree bit for bit."""
    xd = to_dev(x)
    y, s = P.mul_mat_vec(t, wd, M, K, xd, act="q8_1", group_sums=True) if with_sums else (None, None)
    y2 = P.mul_mat_vec(t, wd, M, K, xd, act="q8_1").cpu().numpy()
    if with_sums:
        assert np.array_equal(y.cpu().numpy().view(np.uint32), y2.view(np.uint32)), "group sums changed y"
        return y2, s.cpu().numpy()
    return y2, None


@pytest.mark.parametrize("tname", ["q4_0", "q8_0"])
def test_config1_single_launch_4096x4096(orc, gpu, tname):
    t = P.TYPES[tname]
    M = K = 4096
    assert P.mul_mat_vec_workspace(t, M, K, 1) == 0  # one launch: each work-group quantizes x itself
    wd, w = weights(t, M, K, 101)
    x = activation(K, 1, 1)
    y, s = run_op(t, wd, M, K, x)
    check(orc, t, w, M, K, x, y, s)


LAYER = [("wq", 4096, 4096), ("wk", 1024, 4096), ("gate", 14336, 4096), ("down", 4096, 14336)]


@pytest.mark.parametrize("ncols", [1, 2, 4, 8])
@pytest.mark.parametrize("shape", LAYER, ids=[s[0] for s in LAYER])
@pytest.mark.parametrize("tname", ["q4_0", "q8_0"])
def test_config2_layer_sweep(orc, gpu, tname, shape, ncols):
    """Each layer matrix at ne11 1..8 through the f32 op (with and without sums) and through a prepared Q8_1
    activation (the decode's form; one column is the register-resident kernel)."""
    t = P.TYPES[tname]
    _, M, K = shape
    wd, w = weights(t, M, K, 200 + M + K)
    x = activation(K, ncols, 10 * ncols + M)
    y, s = run_op(t, wd, M, K, x)
    check(orc, t, w, M, K, x, y, s)
    q = P.quantize_q8_1(to_dev(x))
    yq, sq = P.mul_mat_vec(t, wd, M, K, q, group_sums=True)
    yq2 = P.mul_mat_vec(t, wd, M, K, q).cpu().numpy()
    assert np.array_equal(yq.cpu().numpy().view(np.uint32), yq2.view(np.uint32))
    check(orc, t, w, M, K, x, yq2, sq.cpu().numpy())


KQUANT = [("q4_K", 14336, 4096, (1, 8)), ("q4_K", 4096, 14336, (1,)), ("q6_K", 128256, 4096, (1,)),
          ("q6_K", 4096, 14336, (1,))]


@pytest.mark.parametrize("case", KQUANT, ids=[f"{c[0]}-{c[1]}x{c[2]}" for c in KQUANT])
def test_config4_kquants(orc, gpu, case):
    """K-quant matrices at full size through the op (Q8_1 pass + kernel): one row per wave at one column (q6_K on
    rows of 4096-multiples with paired sub-blocks), the int8 matrix cores at 8 columns of q4_K 14336x4096."""
    tname, M, K, cols = case
    t = P.TYPES[tname]
    wd, w = weights(t, M, K, 400 + M)
    for ncols in cols:
        x = activation(K, ncols, 40 + ncols)
        y, s = run_op(t, wd, M, K, x)
        check(orc, t, w, M, K, x, y, s)


H16 = [(n, M, K) for n in ("q4_0", "q8_0", "q4_K", "q6_K") for M, K in ((4096, 4096), (14336, 4096))]


@pytest.mark.parametrize("case", H16, ids=[f"{c[0]}-{c[1]}x{c[2]}" for c in H16])
def test_h16_config_shapes(orc, gpu, case):
    """The h16 (MMVH) path where it runs 64 threads per row: within 1e-3 of FP64, 1e-5 of the h16 model, and the
    same bits through a prepared activation."""
    tname, M, K = case
    t = P.TYPES[tname]
    wd, w = weights(t, M, K, 500 + M)
    for ncols in (1, 4, 8):
        x = activation(K, ncols, 50 + ncols)
        y = P.mul_mat_vec(t, wd, M, K, to_dev(x), act="h16").cpu().numpy()
        check(orc, t, w, M, K, x, y, mode="h16")
        y2 = P.mul_mat_vec(t, wd, M, K, P.prepare_h16(to_dev(x))).cpu().numpy()
        assert np.array_equal(y2.view(np.uint32), y.view(np.uint32))


# ------------------------------------------------------------------------------------------------ 8B decode
def test_decode_8b_step_equals_composed_ops(gpu):
    """The 32-layer Llama-3-8B-shape Q4_0 model: 600 prompt positions through the captured step (a multi-split
    attention plan), then three steps, each bit-identical (logits, token, every layer's KV cache, state) to the
    same step composed from the entry points."""
    import torch

    from p100_amd import llama

    from test_gpu_decode import compose_step

    hp = llama.hparams(768)
    model = llama.LlamaModel(hp, device="cuda", seed=21)
    n_prompt = 600
    dec = llama.Decoder(model, max_prompt=n_prompt)
    prompt = torch.randint(0, hp.n_vocab, (n_prompt,), generator=torch.Generator().manual_seed(21)).tolist()
    dec.reset(prompt)
    dec.run(n_prompt)
    torch.cuda.synchronize()
    print(f"[decode_8b] {n_prompt} positions decoded; comparing 3 steps", flush=True)
    for pos in range(n_prompt, n_prompt + 3):
        tok = int(dec.tokens[pos].item())
        caches = [(L["k_cache"].clone(), L["v_cache"].clone()) for L in model.layers]
        want_logits, want_tok = compose_step(model, tok, pos, caches)
        dec.step()
        assert torch.equal(dec.logits, want_logits), pos
        assert int(dec.tokens[pos + 1].item()) == want_tok, pos
        for li, ((kc, vc), L) in enumerate(zip(caches, model.layers)):
            assert torch.equal(L["k_cache"], kc) and torch.equal(L["v_cache"], vc), (pos, li)
        assert dec.state.tolist()[:3] == [pos + 1, n_prompt, pos + 1]
    del dec, model
    torch.cuda.empty_cache()


def _mv_check(orc, t, w_dev, M, K, h, y, cache={}):
    """y (GPU mat-vec of the Q8_1 of h, one column) against the oracle's Q8_1 mat-vec of the same f32 h."""
    key = (w_dev.data_ptr(), M, K)
    if key not in cache:
        w = w_dev.cpu().numpy()
        cache[key] = (w, orc.weight_norms(t, w, M, K))
    w, wn = cache[key]
    x = np.ascontiguousarray(h, np.float32).reshape(1, K)
    ref = orc.mul_mat_vec(t, w, M, K, x)[0].astype(np.float64)
    scale = np.linalg.norm(x.astype(np.float64)) * wn
    err = np.abs(y.astype(np.float64) - ref) / np.where(scale > 0, scale, 1.0)
    assert err.max() <= 1e-5, err.max()


def test_decode_8b_layer_ops_match_reference(orc, gpu):
    """One decode layer plus the output head at the 8B dimensions (4096 wide, FFN 14336, 32/8 heads of 128, vocab
    128256), op by op for 4 positions, each op fed the GPU's own inputs (so no rounding difference is carried from
    one op into the next): embedding rows bit-exact; norms and SwiGLU against FP64 with their Q8_1 bit-exact; every
    mat-vec (q/k/v 6144x4096, o 4096x4096, gate/up 28672x4096, down 4096x14336, output 128256x4096) against the
    oracle within 1e-5 |w||x|; RoPE against FP64; attention over the GPU's cache against the FP64 reference within
    tolerance.h. The decode step equals this composition bit for bit (test_decode_8b_step_equals_composed_ops)."""
    import torch

    from p100_amd import llama

    from test_gpu_decode import assert_q81_matches, deq_rows, rope_ref

    hp = llama.hparams(64, n_layer=1)
    model = llama.LlamaModel(hp, device="cuda", seed=5)
    E, F, H, HKV, d = hp.n_embd, hp.n_ff, hp.n_head, hp.n_head_kv, hp.head_dim
    kv = HKV * d
    t = hp.wtype
    L = model.layers[0]
    kc, vc = L["k_cache"].clone(), L["v_cache"].clone()
    emb = model.tok_embd.cpu().numpy()
    p = P.AttnParams(1, H, HKV, 1, hp.n_ctx, d, d, 0.0, 0.0, False)

    def norm64(x, w):
        x64 = x.astype(np.float64)
        return x64 / np.sqrt(np.mean(x64 * x64) + hp.rms_eps) * w.astype(np.float64)

    def dev(v):
        return torch.tensor([v], dtype=torch.int32, device="cuda")

    an, fn_, on = (L["attn_norm"].cpu().numpy(), L["ffn_norm"].cpu().numpy(), model.output_norm.cpu().numpy())
    for pos, tok in enumerate([128000, 9906, 11, 1917]):
        x = P.get_rows(hp.embd_type, model.tok_embd, hp.n_vocab, E, dev(tok))
        xn = x.cpu().numpy()
        assert np.array_equal(xn, deq_rows(hp.embd_type, emb[tok:tok + 1])[0])
        act, h = P.rms_norm_q8_1(x, L["attn_norm"], hp.rms_eps, want_h=True)
        hn = h.cpu().numpy()
        ref = norm64(xn, an)
        assert np.max(np.abs(hn - ref)) <= 2e-6 * np.max(np.abs(ref))
        assert_q81_matches(orc, act, hn)
        qkv = P.mul_mat_vec(t, L["wqkv"], E + 2 * kv, E, act)[0]
        _mv_check(orc, t, L["wqkv"], E + 2 * kv, E, hn, qkv.cpu().numpy())
        qkn = qkv.cpu().numpy()
        qr = P.rope_kv_append(qkv[:E].reshape(H, d), qkv[E:E + kv].reshape(HKV, d), qkv[E + kv:].reshape(HKV, d),
                              kc, vc, dev(pos), rope_base=hp.rope_base)
        rq = rope_ref(qkn[:E].reshape(H, d), pos, hp.rope_base)
        assert np.max(np.abs(qr.cpu().numpy() - rq)) <= 1e-4 * np.max(np.abs(rq)) + 1e-6
        rk = rope_ref(qkn[E:E + kv].reshape(HKV, d), pos, hp.rope_base)
        got_k = kc[:, pos].float().cpu().numpy()
        assert np.all(np.abs(got_k - rk) <= 1e-3 * np.abs(rk) + 1e-4 * np.max(np.abs(rk)))
        assert np.array_equal(vc[:, pos].cpu().numpy(), qkn[E + kv:].reshape(HKV, d).astype(np.float16))
        o, lse = P.flash_attn_decode(p, qr.reshape(-1), kc, vc, kv_len=dev(pos + 1))
        pm = orc.AttnParams(1, H, HKV, 1, pos + 1, d, d, 0.0, 0.0, False)
        ref_o, ref_l = orc.attention_reference(pm, qr.cpu().numpy().ravel(),
                                               kc[:, :pos + 1].float().cpu().numpy(),
                                               vc[:, :pos + 1].float().cpu().numpy())
        on_ = o.cpu().numpy()
        err = np.abs(on_.astype(np.float64) - ref_o)
        assert not (err > 1e-3 + 2e-3 * np.abs(ref_o)).any() and err.max() / np.abs(ref_o).max() <= 2e-3
        assert (np.abs(lse.cpu().numpy() - ref_l) <= 1e-3).all()
        y = P.mul_mat_vec(t, L["wo"], E, E, P.quantize_q8_1(o.reshape(1, E)))[0]
        _mv_check(orc, t, L["wo"], E, E, on_, y.cpu().numpy())
        act, h = P.rms_norm_q8_1(x, L["ffn_norm"], hp.rms_eps, add=y, want_h=True)
        x_res = xn + y.cpu().numpy()
        assert np.array_equal(x.cpu().numpy(), x_res)  # the residual add is one fp32 add
        hn = h.cpu().numpy()
        ref = norm64(x_res, fn_)
        assert np.max(np.abs(hn - ref)) <= 2e-6 * np.max(np.abs(ref))
        assert_q81_matches(orc, act, hn)
        gu = P.mul_mat_vec(t, L["w_gate_up"], 2 * F, E, act)[0]
        _mv_check(orc, t, L["w_gate_up"], 2 * F, E, hn, gu.cpu().numpy())
        act, h = P.swiglu_q8_1(gu[:F], gu[F:], want_h=True)
        g64 = gu.cpu().numpy().astype(np.float64)
        ref = g64[:F] / (1.0 + np.exp(-g64[:F])) * g64[F:]
        hn = h.cpu().numpy()
        assert np.all(np.abs(hn - ref) <= 1e-6 * np.abs(ref) + 1e-30)
        assert_q81_matches(orc, act, hn)
        y2 = P.mul_mat_vec(t, L["w_down"], E, F, act)[0]
        _mv_check(orc, t, L["w_down"], E, F, hn, y2.cpu().numpy())
        act, h = P.rms_norm_q8_1(x, model.output_norm, hp.rms_eps, add=y2, want_h=True)
        hn = h.cpu().numpy()
        x_res = x_res + y2.cpu().numpy()
        ref = norm64(x_res, on)
        assert np.max(np.abs(hn - ref)) <= 2e-6 * np.max(np.abs(ref))
        logits = P.mul_mat_vec(hp.output_type, model.output, hp.n_vocab, E, act)[0]
        _mv_check(orc, hp.output_type, model.output, hp.n_vocab, E, hn, logits.cpu().numpy())
        print(f"[decode_8b_ops] position {pos} checked", flush=True)
    del model
    torch.cuda.empty_cache()


def test_decode_8b_layer_matches_reference(orc, gpu):
    """End to end at the 8B dimensions (one layer, vocab 128256) against the CPU restatement, 8 positions. Each
    op agrees with its reference to the bars above, but the two sides round differently in the last fp32 bit, and
    where that straddles a Q8_1 rounding step one activation code moves; with 4096- and 14336-wide activations
    such steps occur at most positions and move the logits by a few percent of their range. So: position 0 (one
    key, attention exact) within 1e-4 of the range, every position within 5e-2, and the greedy choice equal to the
    reference's wherever its margin exceeds 10 % of the range. A wiring error (head mapping, RoPE, GQA, residual)
    moves them by O(1)."""
    import torch

    from p100_amd import llama

    from test_gpu_decode import RefLlama

    hp = llama.hparams(64, n_layer=1)
    model = llama.LlamaModel(hp, device="cuda", seed=5)
    dec = llama.Decoder(model, max_prompt=4)
    ref = RefLlama(orc, model)
    prompt = [128000, 9906, 11, 1917]
    dec.reset(prompt)
    toks = list(prompt)
    errs = []
    for pos in range(8):
        for li, L in enumerate(model.layers):
            ref.kc[li, :, :pos] = L["k_cache"][:, :pos].cpu().numpy()
            ref.vc[li, :, :pos] = L["v_cache"][:, :pos].cpu().numpy()
        dec.step()
        got = dec.logits.cpu().numpy()
        want = ref.step(toks[pos], pos)
        scale = np.max(np.abs(want))
        err = float(np.max(np.abs(got - want)) / scale)
        errs.append(err)
        assert err <= 5e-2, (pos, err)
        nxt = int(dec.tokens[pos + 1].item())
        assert nxt == int(np.argmax(got))
        top2 = np.sort(want)[-2:]
        if top2[1] - top2[0] > 0.1 * scale:
            assert nxt == int(np.argmax(want)), pos
        if pos + 1 >= len(toks):
            toks.append(nxt)
    print(f"[decode_8b_layer] logit errors / range: {['%.1e' % e for e in errs]}", flush=True)
    assert errs[0] <= 1e-4, errs
    del dec, model
    torch.cuda.empty_cache()
