"""Seeded synthetic inputs of the BASELINE configurations.

Weights are generated directly as GGUF block bytes (numpy PCG64 streams, so
the same seed gives the same bytes on every host):
  q8_0  quants uniform in [-127, 127], d = fp16(|N(0,1)| * 0.02/127)
  q4_0  nibbles uniform in 0..15,     d = fp16(|N(0,1)| * 0.02/8)
  q2_K / q3_K / q4_K / q5_K / q6_K  every quant, scale and hmask bit uniform random;
        d and dmin = fp16(|N(0,1)| * 1e-4) so that they are finite.
  tq2_0 every 2-bit field uniform in 0..3 (value -1..2), d = fp16(|N(0,1)| * 0.02).
  f16 / bf16  N(0, 0.02) values, rounded to f16 / truncated to bf16.
Activations x ~ N(0,1) in fp32.
"""
from __future__ import annotations

import numpy as np

from . import BF16, BLCK, F16, Q2_K, Q3_K, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, SIZE, TQ2_0

# byte offsets of the fp16 scale fields inside each block (g4run.h:107-118)
_SCALE_FIELDS = {Q8_0: (0,), Q4_0: (0,), Q2_K: (80, 82), Q3_K: (108,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,), TQ2_0: (64,)}
_SCALE_MUL = {Q8_0: 0.02 / 127, Q4_0: 0.02 / 8, Q2_K: 1e-4, Q3_K: 1e-4, Q4_K: 1e-4, Q5_K: 1e-4, Q6_K: 1e-5, TQ2_0: 0.02}


def _fp16_bits(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float32).astype(np.float16).view(np.uint16)


def weights(qtype: int, nrows: int, ncols: int, seed: int) -> np.ndarray:
    """GGUF rows [nrows, row_bytes] of a synthetic weight matrix."""
    rng = np.random.default_rng(seed)
    if qtype in (F16, BF16):
        wf = (rng.standard_normal((nrows, ncols)) * 0.02).astype(np.float32)
        w = wf.astype(np.float16).view(np.uint16) if qtype == F16 else (wf.view(np.uint32) >> 16).astype(np.uint16)
        return np.ascontiguousarray(w).view(np.uint8).reshape(nrows, 2 * ncols)
    nb = ncols // BLCK[qtype]
    bs = SIZE[qtype]
    w = rng.integers(0, 256, size=(nrows, nb, bs), dtype=np.uint8)
    if qtype == Q8_0:
        w[:, :, 2:] = rng.integers(-127, 128, size=(nrows, nb, 32), dtype=np.int8).view(np.uint8)
    for off in _SCALE_FIELDS[qtype]:
        h = _fp16_bits(np.abs(rng.standard_normal((nrows, nb))) * _SCALE_MUL[qtype])
        w[:, :, off] = (h & 0xFF).astype(np.uint8)
        w[:, :, off + 1] = (h >> 8).astype(np.uint8)
    return w.reshape(nrows, nb * bs)


def activations(nb: int, ncols: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((nb, ncols)).astype(np.float32)


# BASELINE.json configs (GEMV shapes: rows x cols)
GEMV_CONFIGS = {
    "q8_0_4096x4096": (Q8_0, 4096, 4096),
    "q4_0_10240x2560": (Q4_0, 10240, 2560),
    "q4_0_2560x10240": (Q4_0, 2560, 10240),
    "q4_K_4096x11008": (Q4_K, 4096, 11008),
    "q3_K_4096x11008": (Q3_K, 4096, 11008),
    "q2_K_4096x11008": (Q2_K, 4096, 11008),
    # beyond BASELINE config 2: the next K-quant formats of the same boundary
    "q5_K_4096x11008": (Q5_K, 4096, 11008),
    "q6_K_4096x11008": (Q6_K, 4096, 11008),
    "tq2_0_4096x11008": (TQ2_0, 4096, 11008),
    "f16_4096x4096": (F16, 4096, 4096),
    "bf16_4096x4096": (BF16, 4096, 4096),
}

SEEDS = {"weights": 1234, "x": 99}


def algorithmic_bytes(qtype: int, nrows: int, ncols: int, nb: int = 1) -> int:
    """Weights + quantized activation + fp32 output, each counted once."""
    from . import act_type, row_size
    return nrows * row_size(qtype, ncols) + nb * row_size(act_type(qtype), ncols) + nb * nrows * 4
