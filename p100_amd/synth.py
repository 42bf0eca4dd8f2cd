"""Synthetic GGUF weights for benchmarks and demos, quantized with torch on any device (GPU for the bench).

* q4_0 / q8_0: the arithmetic of ggml's reference quantizers (quantize_row_q4_0_ref / quantize_row_q8_0_ref,
  llama.cpp @ 79e2e74): q4_0 d = (signed value of largest magnitude) / -8, q = min(15, trunc(x/d + 8.5));
  q8_0 d = amax / 127, q = round(x/d); d stored as fp16.
* q4_K / q6_K: simple max-based quantizers (NOT ggml's iterative scale search), producing valid blocks:
  q4_K per 32 scale = (max - min)/15 with min clipped to <= 0, six-bit codes against d = max scale/63 and
  dmin = max(-min)/63; q6_K per 16 scale = amax/31 with int8 codes against d = max scale/127.
Each returns a uint8 tensor [rows, row_bytes] in the GGUF block layout.
"""
from __future__ import annotations

import torch


def _round_away(t: torch.Tensor) -> torch.Tensor:
    """Round half away from zero (C lround / roundf), unlike torch.round's half to even."""
    return torch.sign(t) * torch.floor(t.abs() + 0.5)


def _fp16_bits(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF


def _u16_bytes(bits: torch.Tensor) -> torch.Tensor:
    return torch.stack([(bits & 255), (bits >> 8) & 255], -1).to(torch.uint8)


def quantize_q4_0(x: torch.Tensor) -> torch.Tensor:
    rows, k = x.shape
    b = x.reshape(rows, k // 32, 32).float()
    idx = b.abs().argmax(-1, keepdim=True)  # first index of the largest magnitude, as the sequential scan
    mx = torch.gather(b, -1, idx).squeeze(-1)
    d = mx / -8.0
    inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
    q = torch.clamp((b * inv.unsqueeze(-1) + 8.5).to(torch.int8).to(torch.int32), max=15)
    packed = (q[..., :16] | (q[..., 16:] << 4)).to(torch.uint8)
    out = torch.cat([_u16_bytes(_fp16_bits(d)), packed], -1)
    return out.reshape(rows, k // 32 * 18)


def quantize_q8_0(x: torch.Tensor) -> torch.Tensor:
    rows, k = x.shape
    b = x.reshape(rows, k // 32, 32).float()
    amax = b.abs().amax(-1)
    d = amax / 127.0
    inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
    r = b * inv.unsqueeze(-1)
    q = torch.sign(r) * torch.floor(r.abs() + 0.5)  # roundf: ties away from zero (|r| <= 127)
    qs = q.to(torch.int8).view(torch.uint8)
    out = torch.cat([_u16_bytes(_fp16_bits(d)), qs], -1)
    return out.reshape(rows, k // 32 * 34)


def quantize_q4_K(x: torch.Tensor) -> torch.Tensor:
    rows, k = x.shape
    b = x.reshape(rows, k // 256, 8, 32).float()
    lo = torch.clamp(b.amin(-1), max=0.0)
    hi = torch.clamp(b.amax(-1), min=0.0)
    scale = (hi - lo) / 15.0
    mins = -lo
    d = (scale.amax(-1) / 63.0).to(torch.float16).float()
    dmin = (mins.amax(-1) / 63.0).to(torch.float16).float()
    sc = torch.where(d.unsqueeze(-1) > 0, _round_away(scale / d.unsqueeze(-1).clamp(min=1e-30)), torch.zeros_like(scale))
    mn = torch.where(dmin.unsqueeze(-1) > 0, _round_away(mins / dmin.unsqueeze(-1).clamp(min=1e-30)),
                     torch.zeros_like(mins))
    sc = sc.clamp(0, 63).to(torch.int32)
    mn = mn.clamp(0, 63).to(torch.int32)
    ds = (d.unsqueeze(-1) * sc).unsqueeze(-1)
    dm = (dmin.unsqueeze(-1) * mn).unsqueeze(-1)
    q = torch.where(ds > 0, _round_away((b + dm) / ds.clamp(min=1e-30)), torch.zeros_like(b)).clamp(0, 15).to(torch.int32)
    s = torch.zeros(rows, k // 256, 12, dtype=torch.int32, device=x.device)
    s[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    s[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    s[..., 8:12] = (sc[..., 4:8] & 15) | ((mn[..., 4:8] & 15) << 4)
    qs = (q[..., 0::2, :] | (q[..., 1::2, :] << 4)).reshape(rows, k // 256, 128)
    out = torch.cat([_u16_bytes(_fp16_bits(d)), _u16_bytes(_fp16_bits(dmin)), s.to(torch.uint8), qs.to(torch.uint8)], -1)
    return out.reshape(rows, k // 256 * 144)


def quantize_q6_K(x: torch.Tensor) -> torch.Tensor:
    rows, k = x.shape
    nb = k // 256
    b = x.reshape(rows, nb, 16, 16).float()
    scale = b.abs().amax(-1) / 31.0
    d = (scale.amax(-1) / 127.0).to(torch.float16).float()
    sc = torch.where(d.unsqueeze(-1) > 0, _round_away(scale / d.unsqueeze(-1).clamp(min=1e-30)),
                     torch.zeros_like(scale)).clamp(max=127).to(torch.int32)
    ds = (d.unsqueeze(-1) * sc).unsqueeze(-1)
    q = (torch.where(ds > 0, _round_away(b / ds.clamp(min=1e-30)), torch.zeros_like(b)).clamp(-32, 31) + 32)
    q = q.to(torch.int32).reshape(rows, nb, 2, 4, 32)  # [half n][k = 32-group][l]
    ql = torch.zeros(rows, nb, 2, 64, dtype=torch.int32, device=x.device)
    ql[..., 0:32] = (q[..., 0, :] & 15) | ((q[..., 2, :] & 15) << 4)
    ql[..., 32:64] = (q[..., 1, :] & 15) | ((q[..., 3, :] & 15) << 4)
    qh = (q[..., 0, :] >> 4) | ((q[..., 1, :] >> 4) << 2) | ((q[..., 2, :] >> 4) << 4) | ((q[..., 3, :] >> 4) << 6)
    out = torch.cat([ql.reshape(rows, nb, 128).to(torch.uint8), qh.reshape(rows, nb, 64).to(torch.uint8),
                     sc.to(torch.int8).view(torch.uint8), _u16_bytes(_fp16_bits(d))], -1)
    return out.reshape(rows, nb * 210)


QUANTIZERS = {2: quantize_q4_0, 8: quantize_q8_0, 12: quantize_q4_K, 14: quantize_q6_K}


def random_weights(wtype: int, rows: int, k: int, std: float = 0.02, generator=None, device="cuda",
                   chunk_rows: int = 4096) -> torch.Tensor:
    """rows x k weights ~ N(0, std) quantized to wtype, generated and quantized in row chunks on `device`."""
    quant = QUANTIZERS[wtype]
    parts = []
    for r0 in range(0, rows, chunk_rows):
        n = min(chunk_rows, rows - r0)
        x = torch.randn((n, k), generator=generator, device=device, dtype=torch.float32) * std
        parts.append(quant(x))
    return torch.cat(parts, 0).contiguous()
