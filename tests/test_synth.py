"""The torch quantizers that make the bench's synthetic GGUF weights produce exactly the oracle's blocks.

The oracle's q4_0 / q8_0 quantizers follow ggml's reference rule and are pinned by the reference's golden mat-vec
rows (tests/test_oracle_qmv.py); q4_K / q6_K are this build's own max-based rules, so here they only have to agree
byte for byte between the two implementations and decode back within one quantization step.
"""
import numpy as np
import pytest
import torch

from p100_amd import synth

TYPES = {2: "q4_0", 8: "q8_0", 12: "q4_K", 14: "q6_K"}


def _rows(k, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((8, k)) * 0.02).astype(np.float32)
    x[0, :32] = 0.0                     # an all-zero block (d = 0)
    x[1, :32] = 0.01                    # constant block: ties for the largest magnitude
    x[2, 5], x[2, 9] = -0.05, 0.05      # equal magnitudes of opposite sign: the first one sets q4_0's sign
    x[3] *= 1e4                         # large values (fp16 scales near their range)
    x[4, ::7] = 0.0
    x[5] = np.abs(x[5])                 # all positive: q4_K min clipped to 0
    x[6] = -np.abs(x[6])
    return x


@pytest.mark.parametrize("wtype", sorted(TYPES), ids=lambda t: TYPES[t])
@pytest.mark.parametrize("k", [256, 1024])
def test_synth_matches_oracle_quantizer(orc, wtype, k):
    x = _rows(k, seed=wtype * 100 + k)
    mine = synth.QUANTIZERS[wtype](torch.from_numpy(x)).numpy()
    ref = np.stack([orc.quantize(wtype, row) for row in x])
    assert mine.shape == ref.shape
    bad = np.argwhere(mine != ref)
    assert bad.size == 0, f"{TYPES[wtype]}: {len(bad)} bytes differ, first at {bad[:4].tolist()}"


def test_random_weights_shape_and_determinism():
    g1, g2 = torch.Generator().manual_seed(7), torch.Generator().manual_seed(7)
    a = synth.random_weights(2, 40, 256, generator=g1, device="cpu", chunk_rows=16)
    b = synth.random_weights(2, 40, 256, generator=g2, device="cpu", chunk_rows=16)
    assert a.dtype == torch.uint8 and tuple(a.shape) == (40, 256 // 32 * 18)
    assert torch.equal(a, b)
