"""p1x_flash_attn_decode_noalloc: the decode attention entry point that allocates nothing (its split partials live
in the library's per-GPU scratch array). Through the C ABI, against the workspace entry points on the same inputs
(the same kernels and plan, so bit for bit) and against the FP64 reference (tolerance.h), on two calls in a row,
the second smaller; shapes whose partials exceed the scratch are refused without a launch."""
import ctypes as C

import numpy as np
import pytest

import p100_amd as P

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("fa_kernel")]


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _inputs(hq, hkv, seq_kv, d, seed):
    import torch

    rng = np.random.default_rng(seed)
    q = _dev(rng.standard_normal(hq * d).astype(np.float32))
    k16 = rng.standard_normal(hkv * seq_kv * d).astype(np.float16)
    v16 = rng.standard_normal(hkv * seq_kv * d).astype(np.float16)
    return q, k16, v16, _dev(k16.view(np.int16)).view(torch.float16), _dev(v16.view(np.int16)).view(torch.float16)


def _noalloc(lib, p, q, k, v, kv_len=None):
    import torch

    rows = p.batch * p.n_head_q * p.seq_q
    o = torch.full((rows * p.d_v,), 7.0, device="cuda")
    lse = torch.full((rows,), 7.0, device="cuda")
    rc = lib.p1x_flash_attn_decode_noalloc(C.byref(p), P._ptr(q), P._ptr(k), P._ptr(v), None, None, P._ptr(kv_len),
                                           P._ptr(o), P._ptr(lse), P._stream(None))
    return rc, o, lse


def test_noalloc_matches_workspace_entry_points(orc, gpu):
    import torch

    lib = gpu
    # 1: the decode configuration at 8192 keys (16 splits); 2: a smaller cache with a device-side length; 3: a
    # single-split plan (no partials).
    cases = [(32, 8, 8192, 128, None, True), (8, 2, 1000, 64, 700, False), (4, 1, 32, 128, None, False)]
    for i, (hq, hkv, seq_kv, d, n, causal) in enumerate(cases):
        p = P.AttnParams(1, hq, hkv, 1, seq_kv, d, d, 0.0, 0.0, causal)
        q, k16, v16, kd, vd = _inputs(hq, hkv, seq_kv, d, 100 + i)
        kv_len = None if n is None else torch.tensor([n], dtype=torch.int32, device="cuda")
        print(f"[noalloc] case {i}: {hq}/{hkv} heads, d {d}, {seq_kv} keys, kv_len {n}", flush=True)
        rc, o, lse = _noalloc(lib, p, q, kd, vd, kv_len)
        assert rc == P.OK, lib.p1x_last_error().decode()
        want_o, want_l = P.flash_attn_decode(p, q, kd, vd, kv_len=kv_len)
        assert torch.equal(o, want_o) and torch.equal(lse, want_l), i
        m = seq_kv if n is None else n
        pm = orc.AttnParams(1, hq, hkv, 1, m, d, d, 0.0, 0.0, causal)
        kk = k16.reshape(hkv, seq_kv, d)[:, :m].astype(np.float32)
        vv = v16.reshape(hkv, seq_kv, d)[:, :m].astype(np.float32)
        ref, ref_l = orc.attention_reference(pm, q.cpu().numpy(), kk, vv)
        on = o.cpu().numpy().astype(np.float64)
        assert (np.abs(on - ref) <= 1e-3 + 2e-3 * np.abs(ref)).all()
        assert (np.abs(lse.cpu().numpy() - ref_l) <= 1e-3).all()


def test_noalloc_refuses_shapes_beyond_its_scratch(gpu):
    lib = gpu
    # 2 query heads over 1 KV head, 255 query rows, d 256: two splits of 2 x 255 rows of 258 floats (1,052,640 bytes)
    p = P.AttnParams(1, 2, 1, 255, 64, 256, 256, 0.0, 0.0, False)
    assert P.flash_attn_decode_workspace(p) > P.FA_NOALLOC_SCRATCH_BYTES
    q, _, _, kd, vd = _inputs(2 * 255, 1, 64, 256, 9)  # never read: the call is refused before any launch
    rc, o, lse = _noalloc(lib, p, q, kd, vd)
    assert rc == P.EUNSUPPORTED and b"scratch" in lib.p1x_last_error()
    assert bool((o == 7.0).all()) and bool((lse == 7.0).all())
