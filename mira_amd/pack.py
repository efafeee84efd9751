"""Host-side layout of int8 weights and activations for the gfx950 kernels.

Done once at compile time.  The int8 values and per-channel scales are the ones
MIRA's quantizer produced (mira/quantize.py:24-31, 110-115); only their byte
order changes:

* activations are NHWC int8 with `c_pad` channels per pixel: a multiple of 16
  so a 16-byte load never straddles two pixels, or exactly 4 for inputs with at
  most 4 channels (the stem layout: one dword per pixel);
* weights are packed as a logical matrix b[n][k] (`n_pad` rows, `k_pad` bytes
  each, zero-filled), with k running over (kh, kw, c) -- the order in which the
  implicit-GEMM loader walks an NHWC input.  The stem layout packs each kernel
  row as 4-tap groups of one dword per tap.  The device stores that matrix
  K-step-major (`device_weights`): [k_pad / 64][n_pad][64], so the 64-byte
  slices of consecutive rows for one K step are contiguous and a 1 KB load
  covers whole 128-byte cache lines.
"""
from __future__ import annotations

import numpy as np

K_STEP = 64    # bytes of K per pipeline step of the contraction kernel
N_STEP = 32    # MFMA block width


def roundup(x: int, m: int) -> int:
    return -(-x // m) * m


def c_pad_for(c: int) -> int:
    """Channels stored per pixel of an int8 NHWC tensor with c real channels."""
    return 4 if c <= 4 else roundup(c, 16)


def row_stride_for(k: int) -> int:
    """Row stride in bytes of a row-major int8 [M, K] activation."""
    return roundup(k, 16)


def pack_matmul(q: np.ndarray) -> np.ndarray:
    """int8 weights q[K, N] (mira/quantize.py axis 1 = output column) -> b[n_pad, k_pad]."""
    k, n = q.shape
    out = np.zeros((roundup(n, N_STEP), roundup(k, K_STEP)), np.int8)
    out[:n, :k] = q.T
    return out


def conv_row_bytes(kw: int) -> int:
    """Stem layout: bytes per kernel row (taps grouped 4 to a 16-byte chunk)."""
    return 16 * ((kw + 3) // 4)


def pack_conv(q: np.ndarray, c_pad: int, min_rows: int = 0) -> np.ndarray:
    """int8 weights q[O, C, KH, KW] (OIHW, axis 0 = output channel) -> b[n_pad, k_pad]
    (n_pad at least min_rows)."""
    o, c, kh, kw = q.shape
    if c_pad == 4:
        rb = conv_row_bytes(kw)
        body = np.zeros((o, kh, rb // 4, 4), np.int8)             # [o, kh, tap slot, channel]
        body[:, :, :kw, :c] = q.transpose(0, 2, 3, 1)
        body = body.reshape(o, kh * rb)
    else:
        body = np.zeros((o, kh, kw, c_pad), np.int8)
        body[..., :c] = q.transpose(0, 2, 3, 1)
        body = body.reshape(o, kh * kw * c_pad)
    out = np.zeros((max(roundup(o, N_STEP), min_rows), roundup(body.shape[1], K_STEP)), np.int8)
    out[:o, :body.shape[1]] = body
    return out


def device_weights(b: np.ndarray) -> np.ndarray:
    """Logical packed weights b[n_pad, k_pad] -> the kernels' byte order [k_pad/64][n_pad][64]."""
    n_pad, k_pad = b.shape
    assert k_pad % K_STEP == 0, "k_pad must be a multiple of the K step"
    return np.ascontiguousarray(b.reshape(n_pad, k_pad // K_STEP, K_STEP).transpose(1, 0, 2))


def combined_scale(x_scale: float, w_scale: np.ndarray) -> np.ndarray:
    """f64(x_scale) * f64(w_scale[n]) per output channel, as mira/ops.py:618/633 forms it."""
    return np.float64(x_scale) * np.asarray(w_scale).astype(np.float64)
