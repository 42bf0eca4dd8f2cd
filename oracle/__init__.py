"""ctypes access to the CPU oracle (liboracle.so) and the reference build (_ref/libp100_ref.so).

TEST INFRASTRUCTURE ONLY. Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg
may import this package, and only to check results (or as the timed CPU baseline). The product path in
``p100_amd`` never does. Function-by-function reference citations are in ``oracle/oracle.h``.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libp100_ref.so"

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
TYPES = {"q4_0": Q4_0, "q8_0": Q8_0, "q4_K": Q4_K, "q6_K": Q6_K}
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
GROUP = {Q4_0: 32, Q8_0: 32, Q4_K: 32, Q6_K: 16}

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


class AttnParams(C.Structure):
    """Mirrors p100::AttnParams (reference include/p100/attention.h:27-40)."""

    _fields_ = [(n, C.c_int) for n in ("batch", "n_head_q", "n_head_kv", "seq_q", "seq_kv", "d_qk", "d_v")] + [
        ("scale", C.c_float), ("softcap", C.c_float), ("causal", C.c_int)]

    def __init__(self, batch=1, n_head_q=1, n_head_kv=1, seq_q=1, seq_kv=1, d_qk=128, d_v=128, scale=0.0,
                 softcap=0.0, causal=False):
        super().__init__(batch, n_head_q, n_head_kv, seq_q, seq_kv, d_qk, d_v, scale, softcap, int(causal))

    def shapes(self):
        """Element counts of q, k, v, o and lse (0 for invalid negative dimensions)."""
        q = max(0, self.batch * self.n_head_q * self.seq_q)
        kv = max(0, self.batch * self.n_head_kv * self.seq_kv)
        return q * max(0, self.d_qk), kv * max(0, self.d_qk), kv * max(0, self.d_v), q * max(0, self.d_v), q


class TiledConfig(C.Structure):
    """Mirrors p100::TiledModelConfig (reference include/p100/attention.h:54-71), same defaults."""

    _fields_ = [("br", C.c_int), ("bc", C.c_int), ("qk_accum_fp16", C.c_int), ("p_fp16", C.c_int),
                ("o_fp16_out", C.c_int), ("qk_scale_in_q", C.c_int), ("qk_q_prescale", C.c_float),
                ("qk_products_fp16", C.c_int), ("qk_half2_chain", C.c_int), ("kq_max_offset", C.c_float),
                ("l_from_unrounded_p", C.c_int), ("o_accum_fp16", C.c_int), ("kv_parallel_blocks", C.c_int),
                ("o_accum_np", C.c_int), ("o_accum_fp16_tile_flush", C.c_int)]

    def __init__(self, br=64, bc=64, qk_accum_fp16=False, p_fp16=True, o_fp16_out=True, **kw):
        defaults = dict(qk_scale_in_q=0, qk_q_prescale=1.0, qk_products_fp16=0, qk_half2_chain=0,
                        kq_max_offset=0.0, l_from_unrounded_p=0, o_accum_fp16=0, kv_parallel_blocks=1,
                        o_accum_np=1, o_accum_fp16_tile_flush=0)
        defaults.update(kw)
        super().__init__(br, bc, int(qk_accum_fp16), int(p_fp16), int(o_fp16_out))
        for k, v in defaults.items():
            setattr(self, k, v if isinstance(v, float) else int(v))


class RowResult(C.Structure):
    _fields_ = [("exact", C.c_double), ("h16_exact", C.c_double), ("weight_norm", C.c_double),
                ("q81", C.c_float), ("h8", C.c_float), ("h16", C.c_float)]


def build(force: bool = False) -> None:
    """Compile liboracle.so (and the reference build when the reference checkout is present)."""
    if force or not LIB_PATH.exists() or not (HERE / "libcpu_ggml.so").exists():
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


class OracleError(ValueError):
    pass


def _load():
    if not LIB_PATH.exists():
        raise FileNotFoundError(f"{LIB_PATH} is not built (run make -C oracle)")
    lib = C.CDLL(str(LIB_PATH))
    sig = {
        "orc_last_error": (C.c_char_p, []),
        "orc_round_to_fp16_f32": (C.c_float, [C.c_float]),
        "orc_round_to_fp16_f64": (C.c_float, [C.c_double]),
        "orc_half_bits": (C.c_uint16, [C.c_float]),
        "orc_half_value": (C.c_float, [C.c_uint16]),
        "orc_round_to_fp16_array": (None, [f32p, f32p, C.c_int64]),
        "orc_block_size": (C.c_int, [C.c_int]),
        "orc_block_bytes": (C.c_int, [C.c_int]),
        "orc_group_size": (C.c_int, [C.c_int]),
        "orc_rng_new": (C.c_void_p, [C.c_uint32]),
        "orc_rng_free": (None, [C.c_void_p]),
        "orc_rng_normal": (None, [C.c_void_p, C.c_float, C.c_float, f32p, C.c_int64]),
        "orc_rng_uniform": (None, [C.c_void_p, C.c_float, C.c_float, f32p, C.c_int64]),
        "orc_random_row": (C.c_int, [C.c_void_p, C.c_int, C.c_int, u8p]),
        "orc_rng_shuffle_positions": (None, [C.c_void_p, C.c_int64, i32p]),
        "orc_prepare_q8_1": (C.c_int, [f32p, C.c_int, i8p, f32p, f32p]),
        "orc_prepare_h16": (C.c_int, [f32p, C.c_int, u16p, f32p, f32p]),
        "orc_evaluate_row": (C.c_int, [C.c_int, u8p, f32p, C.c_int, C.POINTER(RowResult), C.c_void_p]),
        "orc_mul_mat_vec": (C.c_int, [C.c_int, u8p, C.c_int64, C.c_int64, C.c_int64, f32p, C.c_int64, C.c_int,
                                      f32p, C.c_void_p, C.c_int]),
        "orc_quantize": (C.c_int, [C.c_int, f32p, C.c_int64, u8p]),
        "orc_weight_norms": (C.c_int, [C.c_int, u8p, C.c_int64, C.c_int64, C.c_int64, f64p, C.c_int]),
        "orc_attn_validate": (C.c_int, [C.POINTER(AttnParams)]),
        "orc_attention_reference": (C.c_int, [C.POINTER(AttnParams), C.c_void_p, C.c_void_p, C.c_void_p,
                                              C.c_void_p, C.c_void_p, C.c_void_p]),
        "orc_attention_tiled": (C.c_int, [C.POINTER(AttnParams), C.POINTER(TiledConfig), C.c_void_p, C.c_void_p,
                                          C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
        "orc_fa_decode_f32": (C.c_int, [C.POINTER(AttnParams), f32p, u16p, u16p, C.c_void_p, f32p, C.c_void_p,
                                        C.c_int]),
        "orc_max_threads": (C.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _check(rc):
    if rc != 0:
        raise OracleError(lib().orc_last_error().decode())


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- fp16
def round_to_fp16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_round_to_fp16_array(x.ravel(), out.ravel(), x.size)
    return out


def round_to_fp16_f64(x: float) -> float:
    return lib().orc_round_to_fp16_f64(float(x))


def half_bits(x: float) -> int:
    return lib().orc_half_bits(float(x))


def half_value(h: int) -> float:
    return lib().orc_half_value(int(h))


# ---------------------------------------------------------------- seeded generators
class Rng:
    """std::mt19937 with libstdc++'s distributions, in the reference tests' call order."""

    def __init__(self, seed: int):
        self._h = lib().orc_rng_new(seed)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_rng_free(self._h)
            self._h = None

    def normal(self, n, mean=0.0, stddev=1.0):
        out = np.empty(n, np.float32)
        lib().orc_rng_normal(self._h, mean, stddev, out, n)
        return out

    def uniform(self, n, lo, hi):
        out = np.empty(n, np.float32)
        lib().orc_rng_uniform(self._h, lo, hi, out, n)
        return out

    def shuffle_positions(self, n):
        out = np.empty(n, np.int32)
        lib().orc_rng_shuffle_positions(self._h, n, out)
        return out

    def random_row(self, wtype, k):
        nb, bb = BLOCK[wtype]
        out = np.empty(k // nb * bb, np.uint8)
        _check(lib().orc_random_row(self._h, wtype, k, out))
        return out


# ---------------------------------------------------------------- mat-vec
def prepare_q8_1(x):
    x = np.ascontiguousarray(x, np.float32)
    k = x.size
    q = np.empty(k, np.int8)
    d = np.empty(k // 32, np.float32)
    s = np.empty(k // 32, np.float32)
    _check(lib().orc_prepare_q8_1(x, k, q, d, s))
    return q, d, s


def prepare_h16(x):
    x = np.ascontiguousarray(x, np.float32)
    k = x.size
    h = np.empty(k, np.uint16)
    sc = np.empty(k // 32, np.float32)
    sm = np.empty(k // 32, np.float32)
    _check(lib().orc_prepare_h16(x, k, h, sc, sm))
    return h, sc, sm


def evaluate_row(wtype, w, x, want_sums=False):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.uint8)
    r = RowResult()
    sums = np.empty(x.size // GROUP[wtype], np.int32) if want_sums else None
    _check(lib().orc_evaluate_row(wtype, w, x, x.size, C.byref(r), _ptr(sums)))
    return (r, sums) if want_sums else r


MODE = {"q81": 0, "h8": 8, "h16": 16, "exact": 64}


def mul_mat_vec(wtype, w, M, K, x, mode="q81", nb01=None, want_sums=False, nthreads=0):
    """ggml MUL_MAT restated: w [M][nb01] bytes, x [ncols][K] f32 -> y [ncols][M] f32."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, K)
    ncols = x.shape[0]
    nb, bb = BLOCK[wtype]
    nb01 = nb01 if nb01 is not None else K // nb * bb
    w = np.ascontiguousarray(w, np.uint8).ravel()
    y = np.empty((ncols, M), np.float32)
    sums = np.empty((ncols, M, K // GROUP[wtype]), np.int32) if want_sums else None
    _check(lib().orc_mul_mat_vec(wtype, w, nb01, M, K, x.ravel(), ncols, MODE[mode], y.ravel(), _ptr(sums),
                                 nthreads))
    return (y, sums) if want_sums else y


def weight_norms(wtype, w, M, K, nb01=None, nthreads=0):
    """||deq(w_row)|| (FP64) of every row: evaluate_row's weight_norm for a whole matrix."""
    nb, bb = BLOCK[wtype]
    nb01 = nb01 if nb01 is not None else K // nb * bb
    w = np.ascontiguousarray(w, np.uint8).ravel()
    out = np.empty(M, np.float64)
    _check(lib().orc_weight_norms(wtype, w, nb01, M, K, out, nthreads))
    return out


def quantize(wtype, x):
    x = np.ascontiguousarray(x, np.float32)
    nb, bb = BLOCK[wtype]
    out = np.empty(x.size // nb * bb, np.uint8)
    _check(lib().orc_quantize(wtype, x.ravel(), x.size, out))
    return out


# ---------------------------------------------------------------- attention
def attention_reference(p: AttnParams, q, k, v, mask=None, want_lse=True):
    nq, nk, nv, no, nl = p.shapes()
    o = np.empty(no, np.float32)
    lse = np.empty(nl, np.float32) if want_lse else None
    arrs = [np.ascontiguousarray(a, np.float32) if a is not None else None for a in (q, k, v, mask)]
    _check(lib().orc_attention_reference(C.byref(p), *map(_ptr, arrs), _ptr(o), _ptr(lse)))
    return o, lse


def attention_tiled(p: AttnParams, cfg: TiledConfig, q, k, v, mask=None, want_lse=True):
    nq, nk, nv, no, nl = p.shapes()
    o = np.empty(no, np.float32)
    lse = np.empty(nl, np.float32) if want_lse else None
    arrs = [np.ascontiguousarray(a, np.float32) if a is not None else None for a in (q, k, v, mask)]
    _check(lib().orc_attention_tiled(C.byref(p), C.byref(cfg), *map(_ptr, arrs), _ptr(o), _ptr(lse)))
    return o, lse


def fa_decode_f32(p: AttnParams, q, k16, v16, mask=None, nthreads=0):
    nq, nk, nv, no, nl = p.shapes()
    o = np.empty(no, np.float32)
    lse = np.empty(nl, np.float32)
    m = np.ascontiguousarray(mask, np.float32) if mask is not None else None
    _check(lib().orc_fa_decode_f32(C.byref(p), np.ascontiguousarray(q, np.float32),
                                   np.ascontiguousarray(k16, np.uint16), np.ascontiguousarray(v16, np.uint16),
                                   _ptr(m), o, _ptr(lse), nthreads))
    return o, lse


# ---------------------------------------------------------------- timed CPU baseline (cpu_ggml.cpp)
CPU_GGML_PATH = HERE / "libcpu_ggml.so"
_cpu = None


def _cpu_lib():
    global _cpu
    if _cpu is None:
        if not CPU_GGML_PATH.exists():
            raise FileNotFoundError(f"{CPU_GGML_PATH} is not built (run make -C oracle)")
        L = C.CDLL(str(CPU_GGML_PATH))
        L.cpu_ggml_uses_vnni.restype, L.cpu_ggml_uses_vnni.argtypes = C.c_int, []
        L.cpu_ggml_force_avx2.restype, L.cpu_ggml_force_avx2.argtypes = None, [C.c_int]
        L.cpu_ggml_mul_mat_q4_0.restype = C.c_int
        L.cpu_ggml_mul_mat_q4_0.argtypes = [u8p, C.c_int64, C.c_int64, C.c_int64, f32p, C.c_int64, f32p, C.c_int]
        L.cpu_ggml_fa_decode.restype = C.c_int
        L.cpu_ggml_fa_decode.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, f32p, u16p, u16p, f32p,
                                         f32p, C.c_int]
        _cpu = L
    return _cpu


def cpu_uses_vnni() -> bool:
    return bool(_cpu_lib().cpu_ggml_uses_vnni())


def cpu_force_avx2(on: bool) -> None:
    """Run the AVX2 block dot even where AVX-512 VNNI exists (both kernels are tested)."""
    _cpu_lib().cpu_ggml_force_avx2(int(on))


def cpu_mul_mat_q4_0(w, M, K, x, nb01=None, nthreads=0):
    """ggml's CPU q4_0 x f32 mat-vec restated with SIMD (Q8_0 activation, int8 block dots): y [ncols, M]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, K)
    nb01 = nb01 if nb01 is not None else K // 32 * 18
    y = np.empty((x.shape[0], M), np.float32)
    if _cpu_lib().cpu_ggml_mul_mat_q4_0(np.ascontiguousarray(w, np.uint8).ravel(), nb01, M, K, x.ravel(),
                                        x.shape[0], y.ravel(), nthreads):
        raise OracleError("cpu_ggml_mul_mat_q4_0: invalid arguments")
    return y


def cpu_fa_decode(n_head_q, n_head_kv, seq_kv, d, q, k16, v16, scale=0.0, nthreads=0):
    """Decode attention (one query row per head, every key visible) on the CPU with FP32 accumulation."""
    scale = scale or 1.0 / np.sqrt(d)
    o = np.empty(n_head_q * d, np.float32)
    lse = np.empty(n_head_q, np.float32)
    if _cpu_lib().cpu_ggml_fa_decode(n_head_q, n_head_kv, seq_kv, d, scale, np.ascontiguousarray(q, np.float32),
                                     np.ascontiguousarray(k16, np.uint16).ravel(),
                                     np.ascontiguousarray(v16, np.uint16).ravel(), o, lse, nthreads):
        raise OracleError("cpu_ggml_fa_decode: invalid arguments")
    return o, lse


def validate(p: AttnParams):
    """Returns '' if valid, else the reference's reason string."""
    rc = lib().orc_attn_validate(C.byref(p))
    return "" if rc == 0 else lib().orc_last_error().decode()


def max_threads() -> int:
    return lib().orc_max_threads()


# ---------------------------------------------------------------- the reference's own build
class Ref:
    """The reference's CPU models compiled from their sources (oracle/_ref); absent without the checkout."""

    def __init__(self):
        if not REF_PATH.exists():
            raise FileNotFoundError(str(REF_PATH))
        L = C.CDLL(str(REF_PATH))
        sig = {
            "ref_last_error": (C.c_char_p, []),
            "ref_round_to_fp16_f32": (C.c_float, [C.c_float]),
            "ref_round_to_fp16_f64": (C.c_float, [C.c_double]),
            "ref_half_bits": (C.c_uint16, [C.c_float]),
            "ref_half_value": (C.c_float, [C.c_uint16]),
            "ref_rng_new": (C.c_void_p, [C.c_uint32]),
            "ref_rng_free": (None, [C.c_void_p]),
            "ref_random_row": (C.c_int, [C.c_void_p, C.c_int, C.c_int, u8p]),
            "ref_prepare": (C.c_int, [f32p, C.c_int, f32p, f32p, f32p, f32p, f32p, i32p]),
            "ref_evaluate": (C.c_int, [C.c_int, u8p, f32p, C.c_int, f64p]),
            "ref_attention_reference": (C.c_int, [C.POINTER(AttnParams)] + [C.c_void_p] * 6),
            "ref_attention_tiled": (C.c_int, [C.POINTER(AttnParams), C.POINTER(TiledConfig)] + [C.c_void_p] * 6),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        self.L = L

    def _check(self, rc):
        if rc != 0:
            raise OracleError(self.L.ref_last_error().decode())

    def random_rows(self, seed, wtype, k, rows):
        r = self.L.ref_rng_new(seed)
        nb, bb = BLOCK[wtype]
        out = np.empty((rows, k // nb * bb), np.uint8)
        try:
            for i in range(rows):
                row = np.empty(k // nb * bb, np.uint8)
                self._check(self.L.ref_random_row(r, wtype, k, row))
                out[i] = row
        finally:
            self.L.ref_rng_free(r)
        return out

    def prepare(self, x):
        x = np.ascontiguousarray(x, np.float32)
        nb = x.size // 32
        scale, s, qd, qs = (np.empty(nb, np.float32) for _ in range(4))
        h = np.empty(x.size, np.float32)
        q = np.empty(x.size, np.int32)
        self._check(self.L.ref_prepare(x, x.size, scale, s, h, qd, qs, q))
        return dict(scale=scale, sum=s, h=h, qd=qd, qsum=qs, q=q)

    def evaluate(self, wtype, w, x):
        out = np.empty(6, np.float64)
        self._check(self.L.ref_evaluate(wtype, np.ascontiguousarray(w, np.uint8), np.ascontiguousarray(x, np.float32),
                                        x.size, out))
        return out

    def attention_reference(self, p, q, k, v, mask=None):
        nq, nk, nv, no, nl = p.shapes()
        o, lse = np.empty(no, np.float32), np.empty(nl, np.float32)
        arrs = [np.ascontiguousarray(a, np.float32) if a is not None else None for a in (q, k, v, mask)]
        self._check(self.L.ref_attention_reference(C.byref(p), *map(_ptr, arrs), _ptr(o), _ptr(lse)))
        return o, lse

    def attention_tiled(self, p, cfg, q, k, v, mask=None):
        nq, nk, nv, no, nl = p.shapes()
        o, lse = np.empty(no, np.float32), np.empty(nl, np.float32)
        arrs = [np.ascontiguousarray(a, np.float32) if a is not None else None for a in (q, k, v, mask)]
        self._check(self.L.ref_attention_tiled(C.byref(p), C.byref(cfg), *map(_ptr, arrs), _ptr(o), _ptr(lse)))
        return o, lse


def ref_available() -> bool:
    return REF_PATH.exists() and os.environ.get("P1X_NO_REF") is None
