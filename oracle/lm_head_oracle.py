"""CPU restatement of the reference's LM-head producer (logits for the last
hidden row) and of the weight formats it reads.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's cpu_baseline leg,
always as the checker / reported baseline and never as the thing measured or
shipped.

Reference path (nimbus-infer-rs):
  Model::logits_last      src/model.rs:317-325  lm_head, else the tied wte
  Mat::gemv_into           src/model.rs:65-86    y[j] = dot(x, Wt[j])
  QuantMatrix::dot_rows_into src/quant.rs:121-161 int8 / int4, per row or group
  simd::dot_f32 / dot_f32_i8 / dot_f32_i4  src/simd.rs:22-67
  QuantMatrix::quantize   src/quant.rs:43-95    symmetric RNE quantization
  round_half_even         src/quant.rs:27-39
  dequantize              src/quant.rs:229-250

The reference sums in f32 in its own SIMD lane order; the restatement
evaluates the same sum exactly (f64 products of f32 values are exact, the
f64 sum of H <= 2^20 of them is within H * 2^-53 of the exact value) and
reports sum |x_h * w_h| so a checker can apply the f32 error bound of any
summation order (gamma_n, Higham, Accuracy and Stability, Thm 3.1).
"""
import numpy as np

FMT_F32, FMT_INT8, FMT_INT4 = 0, 8, 4


def round_half_even(x):
    """quant.rs:27-39 on f32 values (np.rint is round-half-to-even)."""
    return np.rint(np.asarray(x, np.float32)).astype(np.float32)


def quantize(w, out_features, in_features, bits, group_size=None):
    """quant.rs:43-95.  Returns (q bytes, scales f32).  Codes are stored biased
    (value + 2^(bits-1)); int4 codes are nibble-packed over the global index
    row*in + k, low nibble first (quant.rs:74-82)."""
    assert bits in (4, 8)
    w = np.asarray(w, np.float32).reshape(out_features, in_features)
    qmax = (1 << (bits - 1)) - 1
    g = group_size or in_features
    assert in_features % g == 0
    groups = in_features // g
    wg = w.reshape(out_features, groups, g)
    amax = np.abs(wg).max(axis=2)
    scale = (amax / np.float32(qmax)).astype(np.float32)   # f32 division (quant.rs:60)
    scale[scale == 0.0] = np.float32(1e-8)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    r = round_half_even((wg * inv[:, :, None]).astype(np.float32)).astype(np.int32)
    r = np.clip(r, -qmax - 1, qmax)
    codes = (r + (1 << (bits - 1))).astype(np.uint8).reshape(-1)
    if bits == 8:
        q = codes
    else:
        n = codes.size
        padded = np.zeros(n + (n & 1), np.uint8)
        padded[:n] = codes
        q = (padded[0::2] & 0x0F) | (padded[1::2] << 4)
    return q.astype(np.uint8), scale.reshape(-1)


def codes(q, bits, numel):
    """The stored code of every weight, in the global row-major index."""
    q = np.asarray(q, np.uint8)
    if bits == 8:
        return q[:numel].astype(np.int32)
    out = np.empty(2 * q.size, np.int32)
    out[0::2] = q & 0x0F
    out[1::2] = q >> 4
    return out[:numel]


def dequantize(q, scales, out_features, in_features, bits, group_size=None):
    """quant.rs:229-250: (code - bias) as f32 times the row's / group's scale."""
    g = group_size or in_features
    c = codes(q, bits, out_features * in_features).reshape(out_features, in_features // g, g)
    bias = 128 if bits == 8 else 8
    s = np.asarray(scales, np.float32).reshape(out_features, in_features // g)
    return ((c - bias).astype(np.float32) * s[:, :, None]).astype(np.float32) \
        .reshape(out_features, in_features)


def effective_weights_f64(fmt, data, scales, V, H, group_size=None):
    """The weight matrix the reference's dot products use, as exact f64 terms:
    dense f32 rows (model.rs:72-78); (code - bias) times the row / group
    scale for int8 / int4 (quant.rs:124-158)."""
    if fmt == FMT_F32:
        return np.asarray(data, np.float32).reshape(V, H).astype(np.float64)
    bits = 8 if fmt == FMT_INT8 else 4
    g = group_size or H
    c = codes(data, bits, V * H).reshape(V, H // g, g).astype(np.float64)
    bias = 128.0 if bits == 8 else 8.0
    s = np.asarray(scales, np.float32).astype(np.float64).reshape(V, H // g)
    return ((c - bias) * s[:, :, None]).reshape(V, H)


def lm_head_logits(hidden, fmt, data, scales, V, H, group_size=None):
    """logits[b][v] = sum_h hidden[b][h] * W[v][h] (model.rs:317-325 for each
    of B last-hidden rows).  Returns (exact f64 logits, f64 sum of |terms|)."""
    x = np.asarray(hidden, np.float32).astype(np.float64).reshape(-1, H)
    w = effective_weights_f64(fmt, data, scales, V, H, group_size)
    return x @ w.T, np.abs(x) @ np.abs(w).T


def f32_bound(abs_terms, H, groups=1):
    """Worst-case |fl32(sum) - sum| for any summation order of H products,
    plus one rounding for the scale product and one per group sum
    (gamma_{H+2+groups} = (H+2+groups) u / (1 - (H+2+groups) u), u = 2^-24)."""
    n = H + 2 + groups
    u = 2.0 ** -24
    return abs_terms * (n * u / (1.0 - n * u)) + 1e-37
