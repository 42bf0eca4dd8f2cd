"""The timed CPU baseline (oracle/cpu_ggml.cpp: ggml's CPU q4_0 x Q8_0 mat-vec and FP32-accumulating decode
attention, restated with AVX-512 VNNI / AVX2) against the oracle, so the baseline the bench reports computes the
same op. Both block-dot kernels run (VNNI where the host has it, AVX2 always)."""
import numpy as np
import pytest


@pytest.fixture(params=["native", "avx2"])
def isa(orc, request):
    orc.cpu_force_avx2(request.param == "avx2")
    yield request.param
    orc.cpu_force_avx2(False)


def test_q4_0_exact_integers(orc, isa):
    """Weights with d = 1 and an activation of integers with |x| max 127 (so the Q8_0 scale is exactly 1):
    every block product is an exact integer and y equals sum (nib - 8) * x exactly."""
    rng = np.random.default_rng(3)
    M, K = 37, 1024
    nib = rng.integers(0, 16, (M, K // 32, 32))
    blk = np.zeros((M, K // 32, 18), np.uint8)
    blk[..., 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[..., 2:] = (nib[..., :16] | (nib[..., 16:] << 4)).astype(np.uint8)
    x = rng.integers(-127, 128, (2, K)).astype(np.float32)
    x[:, ::32] = 127  # amax 127 in every block
    y = orc.cpu_mul_mat_q4_0(blk.reshape(M, -1), M, K, x)
    want = (x.astype(np.int64) @ (nib.reshape(M, K) - 8).T.astype(np.int64)).astype(np.float32)
    assert np.array_equal(y, want)


def test_q4_0_matches_oracle(orc, isa):
    """N(0, 0.02) weights with ggml's q4_0 quantizer, x ~ N(0, 1): within the mat-vec budget of FP64
    (|y - exact| <= 1e-3 ||w|| ||x||). (Q8_0 carries the activation's rounding error into the -8 nibble offset,
    where the Q8_1 path uses the exact block sum s, so the two differ by up to a few 1e-4 |w||x|.)"""
    rng = np.random.default_rng(4)
    M, K = 300, 4096
    w = np.stack([orc.quantize(orc.Q4_0, (rng.standard_normal(K) * 0.02).astype(np.float32)) for _ in range(M)])
    x = rng.standard_normal((3, K)).astype(np.float32)
    y = orc.cpu_mul_mat_q4_0(w, M, K, x)
    exact = orc.mul_mat_vec(orc.Q4_0, w, M, K, x, mode="exact").astype(np.float64)
    scale = np.outer(np.linalg.norm(x, axis=1), orc.weight_norms(orc.Q4_0, w, M, K))
    assert (np.abs(y - exact) / scale).max() <= 1e-3


def test_fa_decode_matches_reference(orc):
    p = orc.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=8192, d_qk=128, d_v=128)
    rng = np.random.default_rng(5)
    q = rng.standard_normal(32 * 128).astype(np.float32)
    k16 = rng.standard_normal(8 * 8192 * 128).astype(np.float16)
    v16 = rng.standard_normal(8 * 8192 * 128).astype(np.float16)
    q[:128] *= 8
    for nthreads in (1, 8):
        o, lse = orc.cpu_fa_decode(32, 8, 8192, 128, q, k16.view(np.uint16), v16.view(np.uint16), nthreads=nthreads)
        ref, ref_lse = orc.attention_reference(p, q, k16.astype(np.float32), v16.astype(np.float32))
        err = np.abs(o.astype(np.float64) - ref)
        assert (err <= 1e-3 + 2e-3 * np.abs(ref)).all() and err.max() / np.abs(ref).max() <= 2e-3
        assert (np.abs(lse.astype(np.float64) - ref_lse) <= 1e-3).all()
