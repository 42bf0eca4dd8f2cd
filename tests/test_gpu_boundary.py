"""GPU parity of the ggml-boundary features of the mat-vec entry points: ggml's ne02/ne03 broadcasting
(third_party/patches/0005-CUDA-half2-mat-vec-for-sm_60-mmvh.patch:271-275, :287-292, :309-321: slice (i2, i3) takes
matrix (i2 / (ne12/ne02), i3 / (ne13/ne03)) and its own src1 columns, dst strides nb1/nb2/nb3), and the AUTO
activation mode driven by p1x_should_use_mmvh. Every slice is checked against the oracle's mat-vec of its own matrix
and columns (bars of tests/test_gpu_matvec.py)."""
import numpy as np
import pytest

import p100_amd as P

pytestmark = pytest.mark.gpu


def to_dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("act", ["q8_1", "h16"])
@pytest.mark.parametrize("tname", ["q4_0", "q8_0", "q4_K", "q6_K"])
def test_broadcast_slices(orc, gpu, tname, act):
    import torch

    t = P.TYPES[tname]
    M, K, ncols = 37, 512, 2
    ne02, ne03, ne12, ne13 = 2, 1, 4, 3  # channel ratio 2, sample ratio 3
    rb = P.row_bytes(t, K)
    nb02 = M * rb + 64  # a gap between matrices
    rng = orc.Rng(900 + t)
    mats = [np.stack([rng.random_row(t, K) for _ in range(M)]) for _ in range(ne02 * ne03)]
    wbuf = np.zeros(nb02 * ne02 * ne03, np.uint8)
    for i, m in enumerate(mats):
        wbuf[i * nb02:i * nb02 + M * rb] = m.ravel()
    x = np.random.default_rng(t).standard_normal((ne13, ne12, ncols, K)).astype(np.float32)
    out = torch.full((ne13, ne12, ncols, M + 3), 7.0, device="cuda")  # padded dst rows: nb1 = 4 (M + 3)
    y = P.mul_mat_vec_batched(t, to_dev(wbuf), M, K, to_dev(x), ne02=ne02, ne03=ne03, nb02=nb02,
                              nb03=nb02 * ne02, act=act, out=out[..., :M])
    got = out.cpu().numpy()
    assert (got[..., M:] == 7.0).all()  # the padding is untouched
    mode = "q81" if act == "q8_1" else "h16"
    for i3 in range(ne13):
        for i2 in range(ne12):
            w = mats[(i3 // (ne13 // ne03)) * ne02 + i2 // (ne12 // ne02)]
            xs = x[i3, i2]
            ref = orc.mul_mat_vec(t, w, M, K, xs, mode=mode)
            exact = orc.mul_mat_vec(t, w, M, K, xs, mode="exact").astype(np.float64)
            scale = np.outer(np.linalg.norm(xs.astype(np.float64), axis=1), orc.weight_norms(t, w, M, K))
            ys = got[i3, i2, :, :M].astype(np.float64)
            assert (np.abs(ys - ref) / scale).max() <= 1e-5, (i3, i2)
            if act == "h16":
                assert (np.abs(ys - exact) / scale).max() <= 1e-3
    assert y.shape == (ne13, ne12, ncols, M)


def test_broadcast_rejects_bad_ratios(gpu):
    import torch

    w = torch.zeros(18 * 4 * 3, dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 3, 1, 32), device="cuda")
    with pytest.raises(ValueError, match="multiples of ne02"):
        P.mul_mat_vec_batched("q4_0", w, 4, 32, x, ne02=2, nb02=72)


def test_auto_mode_follows_the_predicate(orc, gpu):
    """act="auto" runs the path p1x_should_use_mmvh names: bit-identical to that path's explicit mode. q4_K rows
    longer than 8192 at 4+ columns take h16 only where the int8 matrix-core form does not take the shape (fewer
    than 4096 rows)."""
    import torch

    from p100_amd import synth

    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    for tname, M, K, n in (("q4_K", 64, 14336, 4), ("q4_K", 64, 4096, 4), ("q4_0", 64, 14336, 8),
                           ("q4_K", 4096, 14336, 4)):
        t = P.TYPES[tname]
        w = synth.random_weights(t, M, K, generator=g)
        x = torch.randn((n, K), device="cuda", generator=g)
        want = "h16" if P.should_use_mmvh(t, M, K, n) else "q8_1"
        assert want == ("h16" if (tname == "q4_K" and K > 8192 and M < 4096) else "q8_1")
        ya = P.mul_mat_vec(t, w, M, K, x, act="auto")
        ye = P.mul_mat_vec(t, w, M, K, x, act=want)
        assert torch.equal(ya, ye), (tname, M, K, n)
