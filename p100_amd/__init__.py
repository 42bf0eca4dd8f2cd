"""MI355X (gfx950) decode hot path: quantized mat-vec and FlashAttention vector decode behind a C ABI.

Python access to ``libp1x.so`` (declared in ``include/p1x.h``) over ctypes, with torch tensors as the device
memory. The functions mirror the reference's operator interfaces for this path:

* ``mul_mat_vec``  - GGML_OP_MUL_MAT with src0 quantized (q4_0 / q8_0 / q4_K / q6_K) and ne11 = 1..8, as
  ggml_cuda_mul_mat_vec_q / ggml_cuda_mul_mat_vec_h (third_party/patches/0005-...-mmvh.patch:344-377);
  act="q8_1" is the integer (MMVQ) path, act="h16" the block-scaled FP16 (MMVH) path.
* ``quantize_q8_1`` / ``prepare_h16`` - the activation preparations (src/reference/qmv_model.cpp:53-71).
* ``flash_attn_decode`` - GGML_OP_FLASH_ATTN_EXT at decode shapes with the contract of
  p100::attention_reference (include/p100/attention.h:9-49): same AttnParams, same layouts, o and lse outputs,
  and ValueError carrying p100::validate's reason for invalid parameters.

There is no CPU fallback: every call runs the HIP kernels, and loading fails loudly without the library or GPU.
"""
from __future__ import annotations

import ctypes as C
import math
import pathlib
from dataclasses import dataclass

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "libp1x.so"

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
TYPES = {"q4_0": Q4_0, "q8_0": Q8_0, "q4_K": Q4_K, "q6_K": Q6_K}
TYPE_NAMES = {v: k for k, v in TYPES.items()}
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}  # (elements, bytes)
GROUP = {Q4_0: 32, Q8_0: 32, Q4_K: 32, Q6_K: 16}  # elements per exported int32 sum
ACT = {"q8_1": 0, "h16": 1, "auto": 2}
OK, EINVAL, EUNSUPPORTED, EHIP, EWORKSPACE = 0, 1, 2, 3, 4
FA_NOALLOC_SCRATCH_BYTES = 1 << 20  # P1X_FA_NOALLOC_SCRATCH_BYTES
EXPORTS = ["p1x_version", "p1x_init", "p1x_last_error", "p1x_quantize_q8_1", "p1x_prepare_h16",
           "p1x_mul_mat_vec_workspace", "p1x_mul_mat_vec", "p1x_mul_mat_vec_q8_1", "p1x_mul_mat_vec_h16",
           "p1x_attn_validate", "p1x_flash_attn_decode_workspace", "p1x_flash_attn_decode",
           "p1x_flash_attn_decode_kvlen", "p1x_round_to_fp16", "p1x_get_rows", "p1x_rms_norm_q8_1", "p1x_rms_norm_mul_mat_vec",
           "p1x_swiglu_q8_1",
           "p1x_rope_kv_append", "p1x_argmax_workspace", "p1x_argmax", "p1x_llama_workspace", "p1x_llama_decode_step",
           "p1x_flash_attn_decode_quant", "p1x_flash_attn_decode_noalloc", "p1x_read_bytes", "p1x_fa_select_kernel",
           "p1x_should_use_mmvh", "p1x_mul_mat_vec_batched_workspace", "p1x_mul_mat_vec_batched"]


class P1XError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"p1x error {code}: {message}")
        self.code = code
        self.message = message


class AttnParams(C.Structure):
    """p100::AttnParams (include/p100/attention.h:27-40): scale 0 means 1/sqrt(d_qk), softcap 0 means off."""

    _fields_ = [(n, C.c_int) for n in ("batch", "n_head_q", "n_head_kv", "seq_q", "seq_kv", "d_qk", "d_v")] + [
        ("scale", C.c_float), ("softcap", C.c_float), ("causal", C.c_int)]

    def __init__(self, batch=1, n_head_q=1, n_head_kv=1, seq_q=1, seq_kv=1, d_qk=128, d_v=128, scale=0.0,
                 softcap=0.0, causal=False):
        super().__init__(batch, n_head_q, n_head_kv, seq_q, seq_kv, d_qk, d_v, scale, softcap, int(causal))

    def effective_scale(self) -> float:
        return 1.0 / math.sqrt(self.d_qk) if self.scale == 0.0 else self.scale


class MMBatch(C.Structure):
    """p1x_mm_batch: ggml broadcasting of a batched mat-vec over dims 2 and 3."""

    _fields_ = [(n, C.c_int64) for n in ("ne02", "ne03", "nb02", "nb03", "ne12", "ne13", "nb1_dst", "nb2_dst",
                                         "nb3_dst")]


class KVStrides(C.Structure):
    """Element strides of K and V (ggml KV-cache views); omit for dense [batch][n_head_kv][seq_kv][d]."""

    _fields_ = [(n, C.c_int64) for n in ("k_row", "k_head", "k_batch", "v_row", "v_head", "v_batch")]


_lib = None


def load():
    """Loads libp1x.so and initialises it on the current device (raises if either is unavailable)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FileNotFoundError(f"{LIB_PATH} is not built (python -m p100_amd.build)")
    lib = C.CDLL(str(LIB_PATH))
    vp, i64, sz = C.c_void_p, C.c_int64, C.c_size_t
    sig = {
        "p1x_version": (C.c_int, []),
        "p1x_init": (C.c_int, []),
        "p1x_last_error": (C.c_char_p, []),
        "p1x_quantize_q8_1": (C.c_int, [vp, vp, vp, i64, i64, vp]),
        "p1x_prepare_h16": (C.c_int, [vp, vp, vp, i64, i64, vp]),
        "p1x_mul_mat_vec_workspace": (sz, [C.c_int, i64, i64, i64, C.c_int]),
        "p1x_mul_mat_vec": (C.c_int, [C.c_int, vp, i64, i64, i64, C.c_int, vp, i64, vp, vp, vp, sz, vp]),
        "p1x_mul_mat_vec_q8_1": (C.c_int, [C.c_int, vp, i64, i64, i64, vp, vp, i64, vp, vp, vp]),
        "p1x_should_use_mmvh": (C.c_int, [C.c_int, i64, i64, i64]),
        "p1x_mul_mat_vec_batched_workspace": (sz, [C.c_int, i64, i64, i64, C.POINTER(MMBatch), C.c_int]),
        "p1x_mul_mat_vec_batched": (C.c_int, [C.c_int, vp, i64, i64, i64, C.POINTER(MMBatch), C.c_int, vp, i64, vp, vp,
                                              sz, vp]),
        "p1x_mul_mat_vec_h16": (C.c_int, [C.c_int, vp, i64, i64, i64, vp, vp, i64, vp, vp]),
        "p1x_attn_validate": (C.c_int, [C.POINTER(AttnParams)]),
        "p1x_flash_attn_decode_workspace": (sz, [C.POINTER(AttnParams)]),
        "p1x_flash_attn_decode": (C.c_int, [C.POINTER(AttnParams), vp, vp, vp, C.POINTER(KVStrides), vp, vp, vp,
                                            vp, sz, vp]),
        "p1x_flash_attn_decode_kvlen": (C.c_int, [C.POINTER(AttnParams), vp, vp, vp, C.POINTER(KVStrides), vp, vp,
                                                  vp, vp, vp, sz, vp]),
        "p1x_flash_attn_decode_quant": (C.c_int, [C.POINTER(AttnParams), C.c_int, vp, vp, vp, C.POINTER(KVStrides),
                                                  vp, vp, vp, vp, vp, sz, vp]),
        "p1x_flash_attn_decode_noalloc": (C.c_int, [C.POINTER(AttnParams), vp, vp, vp, C.POINTER(KVStrides), vp, vp,
                                                    vp, vp, vp]),
        "p1x_read_bytes": (C.c_int, [vp, sz, vp, C.c_int, vp]),
        "p1x_fa_select_kernel": (C.c_int, [C.c_int]),
        "p1x_round_to_fp16": (C.c_int, [vp, vp, i64, vp]),
        "p1x_get_rows": (C.c_int, [C.c_int, vp, i64, i64, i64, vp, vp, vp]),
        "p1x_rms_norm_q8_1": (C.c_int, [vp, vp, vp, i64, C.c_float, vp, vp, vp, vp]),
        "p1x_rms_norm_mul_mat_vec": (C.c_int, [C.c_int, vp, i64, i64, i64, vp, vp, C.c_float, vp, vp]),
        "p1x_swiglu_q8_1": (C.c_int, [vp, vp, i64, vp, vp, vp, vp]),
        "p1x_rope_kv_append": (C.c_int, [vp, vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, C.c_float, vp]),
        "p1x_argmax_workspace": (sz, [i64]),
        "p1x_argmax": (C.c_int, [vp, i64, vp, vp, sz, vp]),
        "p1x_llama_workspace": (sz, [vp]),
        "p1x_llama_decode_step": (C.c_int, [vp, vp, vp, vp, vp, vp, sz, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    _lib = lib
    rc = lib.p1x_init()
    if rc != OK:
        _lib = None
        raise P1XError(rc, lib.p1x_last_error().decode())
    return lib


def load_symbols_only():
    """Opens the library and resolves every exported entry point without touching a GPU."""
    lib = C.CDLL(str(LIB_PATH))
    return {name: getattr(lib, name) for name in EXPORTS}


def _check(rc):
    if rc != OK:
        msg = _lib.p1x_last_error().decode()
        if rc == EINVAL:
            raise ValueError(msg)
        raise P1XError(rc, msg)


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _params(p) -> AttnParams:
    """Accepts AttnParams or any object with the same fields (e.g. the oracle's mirror of the struct)."""
    if isinstance(p, AttnParams):
        return p
    return AttnParams(p.batch, p.n_head_q, p.n_head_kv, p.seq_q, p.seq_kv, p.d_qk, p.d_v, p.scale, p.softcap,
                      bool(p.causal))


def _stream(stream):
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


# ------------------------------------------------------------------------------------------------ mat-vec
@dataclass
class Q81:
    """Q8_1 activation in this library's layout: qs int8 [ncols, K], ds float32 [ncols, K/32, 4] (d, s, isum, 0)."""
    qs: "object"
    ds: "object"


@dataclass
class H16:
    """h16 activation: h fp16 bits as int16 [ncols, K] (permuted 0,2,1,3), meta float32 [ncols, K/32, 2]."""
    h: "object"
    meta: "object"


def quantize_q8_1(x, stream=None) -> Q81:
    import torch

    lib = load()
    x = x.contiguous()
    ncols, K = (1, x.shape[0]) if x.dim() == 1 else x.shape
    qs = torch.empty((ncols, K), dtype=torch.int8, device=x.device)
    ds = torch.empty((ncols, K // 32, 4), dtype=torch.float32, device=x.device)
    _check(lib.p1x_quantize_q8_1(_ptr(x), _ptr(qs), _ptr(ds), K, ncols, _stream(stream)))
    return Q81(qs, ds)


def prepare_h16(x, stream=None) -> H16:
    import torch

    lib = load()
    x = x.contiguous()
    ncols, K = (1, x.shape[0]) if x.dim() == 1 else x.shape
    h = torch.empty((ncols, K), dtype=torch.int16, device=x.device)
    meta = torch.empty((ncols, K // 32, 2), dtype=torch.float32, device=x.device)
    _check(lib.p1x_prepare_h16(_ptr(x), _ptr(h), _ptr(meta), K, ncols, _stream(stream)))
    return H16(h, meta)


def row_bytes(wtype: int, K: int) -> int:
    n, b = BLOCK[wtype]
    return K // n * b


def mul_mat_vec(wtype, w, M, K, x, act="q8_1", nb01=None, group_sums=False, out=None, workspace=None,
                stream=None):
    """dst[ncols, M] = src1[ncols, K] @ deq(src0[M, K])^T.

    w: uint8 device tensor holding M rows of GGUF blocks with row stride nb01 bytes; x: float32 [ncols, K]
    (ncols 1..8; 1..16 with act="q8_1") or a prepared Q81 / H16 activation. Returns y (and the int32 group sums [ncols, M, K/G] when
    group_sums=True, Q8_1 only).
    """
    import torch

    lib = load()
    wtype = TYPES.get(wtype, wtype)
    if nb01 is None:
        nb01 = row_bytes(wtype, K) if wtype in BLOCK else 0  # unknown types are rejected by the library
    if group_sums and wtype not in GROUP:
        raise P1XError(EUNSUPPORTED, f"unsupported weight type {wtype}")
    s = _stream(stream)
    if isinstance(x, Q81):
        ncols = x.qs.shape[0]
    elif isinstance(x, H16):
        ncols = x.h.shape[0]
    else:
        x = x.contiguous()
        ncols = 1 if x.dim() == 1 else x.shape[0]
    dev = w.device
    y = out if out is not None else torch.empty((ncols, M), dtype=torch.float32, device=dev)
    gs = None
    if group_sums:
        gs = torch.empty((ncols, M, K // GROUP[wtype]), dtype=torch.int32, device=dev)
    if isinstance(x, Q81):
        _check(lib.p1x_mul_mat_vec_q8_1(wtype, _ptr(w), nb01, M, K, _ptr(x.qs), _ptr(x.ds), ncols, _ptr(y),
                                        _ptr(gs), s))
    elif isinstance(x, H16):
        if group_sums:
            raise ValueError("group sums exist only for the Q8_1 activation mode")
        _check(lib.p1x_mul_mat_vec_h16(wtype, _ptr(w), nb01, M, K, _ptr(x.h), _ptr(x.meta), ncols, _ptr(y), s))
    else:
        mode = ACT[act]
        need = lib.p1x_mul_mat_vec_workspace(wtype, M, K, ncols, mode)
        ws = workspace if workspace is not None else torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        _check(lib.p1x_mul_mat_vec(wtype, _ptr(w), nb01, M, K, mode, _ptr(x), ncols, _ptr(y), _ptr(gs), _ptr(ws),
                                   ws.numel(), s))
    return (y, gs) if group_sums else y


def should_use_mmvh(wtype, M, K, ncols) -> bool:
    """ggml_cuda_should_use_mmvh's counterpart: the activation path act="auto" takes for this shape."""
    return bool(load().p1x_should_use_mmvh(TYPES.get(wtype, wtype), M, K, ncols))


def mul_mat_vec_batched(wtype, w, M, K, x, ne02=1, ne03=1, nb02=0, nb03=0, act="q8_1", nb01=None, out=None,
                        stream=None):
    """GGML_OP_MUL_MAT with broadcasting: w holds ne02 x ne03 matrices (byte strides nb02 / nb03), x is float32
    [ne13, ne12, ncols, K]; returns y [ne13, ne12, ncols, M] (or writes `out`, same layout)."""
    import torch

    lib = load()
    wtype = TYPES.get(wtype, wtype)
    if nb01 is None:
        nb01 = row_bytes(wtype, K) if wtype in BLOCK else 0
    x = x.contiguous()
    ne13, ne12, ncols = x.shape[0], x.shape[1], x.shape[2]
    y = out if out is not None else torch.empty((ne13, ne12, ncols, M), dtype=torch.float32, device=w.device)
    b = MMBatch(ne02, ne03, nb02, nb03, ne12, ne13, y.stride(2) * 4, y.stride(1) * 4, y.stride(0) * 4)
    mode = ACT[act]
    need = lib.p1x_mul_mat_vec_batched_workspace(wtype, M, K, ncols, C.byref(b), mode)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=w.device)
    _check(lib.p1x_mul_mat_vec_batched(wtype, _ptr(w), nb01, M, K, C.byref(b), mode, _ptr(x), ncols, _ptr(y),
                                       _ptr(ws), ws.numel(), _stream(stream)))
    return y


def mul_mat_vec_workspace(wtype, M, K, ncols, act="q8_1") -> int:
    return load().p1x_mul_mat_vec_workspace(TYPES.get(wtype, wtype), M, K, ncols, ACT[act])


# ------------------------------------------------------------------------------------------------ attention
def validate(p: AttnParams) -> str:
    """'' if p is valid, else p100::validate's reason string."""
    lib = load()
    p = _params(p)
    return "" if lib.p1x_attn_validate(C.byref(p)) == OK else lib.p1x_last_error().decode()


FA_KERNEL = {"auto": 0, "split": 1, "mc": 2}  # P1X_FA_KERNEL_AUTO / _SPLIT / _MC


def fa_select_kernel(kernel: str) -> None:
    """The decode attention's first-pass kernel for the process: "auto", "split" (vector) or "mc" (matrix cores)."""
    lib = load()
    if lib.p1x_fa_select_kernel(FA_KERNEL[kernel]) != OK:
        raise ValueError(lib.p1x_last_error().decode())


def flash_attn_decode_workspace(p: AttnParams) -> int:
    """Bytes of device workspace for flash_attn_decode (0 when the KV range is not split)."""
    return load().p1x_flash_attn_decode_workspace(C.byref(_params(p)))


def flash_attn_decode(p: AttnParams, q, k, v, mask=None, strides: KVStrides | None = None, want_lse=True, out=None,
                      lse=None, workspace=None, stream=None, kv_len=None):
    """o, lse = attention(q, k, v) with the contract of p100::attention_reference.

    q float32 [batch, n_head_q, seq_q, d]; k, v float16 [batch, n_head_kv, seq_kv, d] (or strided views with
    ``strides``); mask optional float32 [seq_q, seq_kv]. Raises ValueError(reason) for invalid parameters.
    kv_len: optional device int32 tensor; when given, only its first element's count of K/V rows is valid (read
    when the kernels run), p.seq_kv being the cache capacity.
    """
    import torch

    lib = load()
    p = _params(p)
    why = validate(p)
    if why:
        raise ValueError(why)
    dev = q.device
    rows = p.batch * p.n_head_q * p.seq_q
    o = out if out is not None else torch.empty(rows * p.d_v, dtype=torch.float32, device=dev)
    l_out = (lse if lse is not None else torch.empty(rows, dtype=torch.float32, device=dev)) if want_lse else None
    need = lib.p1x_flash_attn_decode_workspace(C.byref(p))
    ws = workspace if workspace is not None else torch.empty(max(need, 16) // 4 + 4, dtype=torch.float32, device=dev)
    if ws.numel() * ws.element_size() < need:
        raise P1XError(EWORKSPACE, f"workspace of {need} bytes required")
    sp = C.byref(strides) if strides is not None else None
    nbytes = ws.numel() * ws.element_size()
    if kv_len is None:
        _check(lib.p1x_flash_attn_decode(C.byref(p), _ptr(q), _ptr(k), _ptr(v), sp, _ptr(mask), _ptr(o), _ptr(l_out),
                                         _ptr(ws), nbytes, _stream(stream)))
    else:
        _check(lib.p1x_flash_attn_decode_kvlen(C.byref(p), _ptr(q), _ptr(k), _ptr(v), sp, _ptr(mask), _ptr(kv_len),
                                               _ptr(o), _ptr(l_out), _ptr(ws), nbytes, _stream(stream)))
    return o, l_out


def flash_attn_decode_quant(p: AttnParams, kv_type, q, k, v, mask=None, byte_strides: KVStrides | None = None,
                            kv_len=None, want_lse=True, out=None, lse=None, workspace=None, stream=None):
    """flash_attn_decode over a q8_0 / q4_0 KV cache: k, v uint8 tensors of GGUF blocks, rows of d_qk / 32 blocks
    ([batch, n_head_kv, seq_kv] rows when dense; otherwise byte_strides)."""
    import torch

    lib = load()
    p = _params(p)
    why = validate(p)
    if why:
        raise ValueError(why)
    dev = q.device
    rows = p.batch * p.n_head_q * p.seq_q
    o = out if out is not None else torch.empty(rows * p.d_v, dtype=torch.float32, device=dev)
    l_out = (lse if lse is not None else torch.empty(rows, dtype=torch.float32, device=dev)) if want_lse else None
    need = lib.p1x_flash_attn_decode_workspace(C.byref(p))
    ws = workspace if workspace is not None else torch.empty(max(need, 16) // 4 + 4, dtype=torch.float32, device=dev)
    sp = C.byref(byte_strides) if byte_strides is not None else None
    _check(lib.p1x_flash_attn_decode_quant(C.byref(p), TYPES.get(kv_type, kv_type), _ptr(q), _ptr(k), _ptr(v), sp,
                                           _ptr(mask), _ptr(kv_len), _ptr(o), _ptr(l_out), _ptr(ws),
                                           ws.numel() * ws.element_size(), _stream(stream)))
    return o, l_out


def round_to_fp16(x, stream=None):
    """The device's fp32 -> fp16 conversion (v_cvt_f16_f32, round to nearest even), as int16 bits."""
    import torch

    lib = load()
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.int16, device=x.device)
    _check(lib.p1x_round_to_fp16(_ptr(x), _ptr(out), x.numel(), _stream(stream)))
    return out


# ------------------------------------------------------------------------------------------------ decode glue
def get_rows(wtype, w, n_rows, K, row, nb01=None, out=None, stream=None):
    """out[K] = dequantized row *row (device int32 tensor) of a q4_0 / q8_0 matrix (ggml GET_ROWS)."""
    import torch

    lib = load()
    wtype = TYPES.get(wtype, wtype)
    nb01 = row_bytes(wtype, K) if nb01 is None else nb01
    y = out if out is not None else torch.empty(K, dtype=torch.float32, device=w.device)
    _check(lib.p1x_get_rows(wtype, _ptr(w), nb01, n_rows, K, _ptr(row), _ptr(y), _stream(stream)))
    return y


def rms_norm_q8_1(x, w, eps=1e-5, add=None, want_h=False, stream=None):
    """x += add (in place, when given); h = x * rsqrt(mean(x^2) + eps) * w; returns Q81(h) (and h)."""
    import torch

    lib = load()
    n = x.numel()
    qs = torch.empty((1, n), dtype=torch.int8, device=x.device)
    ds = torch.empty((1, n // 32, 4), dtype=torch.float32, device=x.device)
    h = torch.empty(n, dtype=torch.float32, device=x.device) if want_h else None
    _check(lib.p1x_rms_norm_q8_1(_ptr(x), _ptr(add), _ptr(w), n, eps, _ptr(qs), _ptr(ds), _ptr(h), _stream(stream)))
    return (Q81(qs, ds), h) if want_h else Q81(qs, ds)


def rms_norm_mul_mat_vec(wtype, w, M, K, x, norm_w, eps=1e-5, nb01=None, out=None, stream=None):
    """y[M] = deq(w) @ Q81(x * rsqrt(mean(x^2) + eps) * norm_w) in one launch (q4_0 / q8_0, K <= 8192): the result
    of rms_norm_q8_1 (no add) then mul_mat_vec on it, bit for bit."""
    import torch

    lib = load()
    wtype = TYPES.get(wtype, wtype)
    if nb01 is None:
        nb01 = row_bytes(wtype, K) if wtype in BLOCK else 0
    y = out if out is not None else torch.empty(M, dtype=torch.float32, device=w.device)
    _check(lib.p1x_rms_norm_mul_mat_vec(wtype, _ptr(w), nb01, M, K, _ptr(x), _ptr(norm_w), eps, _ptr(y),
                                        _stream(stream)))
    return y


def swiglu_q8_1(gate, up, want_h=False, stream=None):
    """h = silu(gate) * up; returns Q81(h) (and h)."""
    import torch

    lib = load()
    n = gate.numel()
    qs = torch.empty((1, n), dtype=torch.int8, device=gate.device)
    ds = torch.empty((1, n // 32, 4), dtype=torch.float32, device=gate.device)
    h = torch.empty(n, dtype=torch.float32, device=gate.device) if want_h else None
    _check(lib.p1x_swiglu_q8_1(_ptr(gate), _ptr(up), n, _ptr(qs), _ptr(ds), _ptr(h), _stream(stream)))
    return (Q81(qs, ds), h) if want_h else Q81(qs, ds)


def rope_kv_append(q, k, v, k_cache, v_cache, pos, rope_base=500000.0, q_out=None, stream=None):
    """RoPE (normal mode) of q [n_head, d] into q_out and of k [n_head_kv, d] into row *pos of k_cache; v into
    row *pos of v_cache. Caches float16 [n_head_kv, n_ctx, d]; pos a device int32 tensor. Returns q_out."""
    import torch

    lib = load()
    n_head, d = q.shape
    n_head_kv, n_ctx = k_cache.shape[0], k_cache.shape[1]
    qo = q_out if q_out is not None else torch.empty_like(q)
    _check(lib.p1x_rope_kv_append(_ptr(q), _ptr(k), _ptr(v), _ptr(qo), _ptr(k_cache), _ptr(v_cache), n_head,
                                  n_head_kv, d, n_ctx, _ptr(pos), rope_base, _stream(stream)))
    return qo


def argmax(x, stream=None):
    """Index of the largest element (first on ties; NaN never wins) as a device int32 tensor of one element."""
    import torch

    lib = load()
    n = x.numel()
    ws = torch.empty(max(lib.p1x_argmax_workspace(n), 8), dtype=torch.uint8, device=x.device)
    out = torch.empty(1, dtype=torch.int32, device=x.device)
    _check(lib.p1x_argmax(_ptr(x), n, _ptr(out), _ptr(ws), ws.numel(), _stream(stream)))
    return out
