"""Pins the LM-head oracle (oracle/lm_head_oracle.py) before GPU logits are
compared against it.

  - the reference's own unit tests as golden vectors: round_half_even
    (quant.rs:269-277), the int8 / grouped int4 round trips and byte counts
    (quant.rs:279-298), dot_row against the dequantized matmul for four
    formats (quant.rs:300-320), and the int8 / int4 dot fixtures with their
    biased-code packing (simd.rs:192-230);
  - brute-force loops over tiny non-square shapes (a transposed operand, a
    wrong scale index or a low/high nibble swap fails them);
  - the f32 error bound used by the GPU tests: f32 sums in several orders lie
    inside it, a one-ulp-per-term slip of the kind a dropped term or wrong
    scale makes does not.
"""
import numpy as np
import pytest

from oracle import lm_head_oracle as lh


def sample_weights(out, inp):
    """quant.rs:258-266: ((i*2654435761) % 1000)/1000 mapped to [-0.05, 0.05)."""
    i = np.arange(out * inp, dtype=np.uint64)
    x = ((i * np.uint64(2654435761)) % np.uint64(1000)).astype(np.float64) / 1000.0
    return ((x * 2.0 - 1.0) * 0.05).astype(np.float32)


def nbytes(q, scales):
    return q.size + scales.size * 4


def test_round_half_even_matches_reference_cases():
    cases = {0.5: 0.0, 1.5: 2.0, 2.5: 2.0, -0.5: -0.0, -1.5: -2.0, 3.5: 4.0}
    for x, want in cases.items():
        assert lh.round_half_even(x) == want


def test_int8_roundtrip_and_bytes():
    w = sample_weights(16, 64)
    q, s = lh.quantize(w, 16, 64, 8)
    assert nbytes(q, s) == 16 * 64 + 16 * 4
    err = np.abs(w - lh.dequantize(q, s, 16, 64, 8).reshape(-1)).max()
    assert err <= s[0] / 2 + 1e-9


def test_int4_grouped_roundtrip_and_bytes():
    w = sample_weights(8, 128)
    q, s = lh.quantize(w, 8, 128, 4, 64)
    assert nbytes(q, s) == 8 * 128 // 2 + 8 * 2 * 4
    err = np.abs(w - lh.dequantize(q, s, 8, 128, 4, 64).reshape(-1)).max()
    assert err <= s[0] / 2 + 1e-9


@pytest.mark.parametrize("bits,group", [(8, None), (4, 32), (8, 48), (4, None)])
def test_dot_rows_match_dequantized_matmul(bits, group):
    w = sample_weights(12, 96)
    x = (np.arange(96, dtype=np.float32) * np.float32(0.02) - np.float32(0.9)).astype(np.float32)
    q, s = lh.quantize(w, 12, 96, bits, group)
    fmt = lh.FMT_INT8 if bits == 8 else lh.FMT_INT4
    got, _ = lh.lm_head_logits(x[None, :], fmt, q, s, 12, 96, group)
    wq = lh.dequantize(q, s, 12, 96, bits, group)
    ref = (wq * x[None, :]).astype(np.float32).sum(axis=1, dtype=np.float32)
    assert np.all(np.abs(got[0] - ref) < 1e-3)


def test_int8_dot_fixture():
    a = np.arange(131, dtype=np.float32) * np.float32(0.125)
    raw = (np.arange(131) * 7) % 255 - 128
    biased = (raw + 128).astype(np.uint8)
    got, _ = lh.lm_head_logits(a[None, :], lh.FMT_INT8, biased, np.ones(1, np.float32), 1, 131)
    assert got[0, 0] == float(np.dot(a.astype(np.float64), raw.astype(np.float64)))


def test_int4_dot_fixture_packing():
    q = ((np.arange(255) * 13) % 16 - 8).astype(np.int32)
    packed = []
    chunk = 0
    for i, v in enumerate(q):
        nib = (v + 8) & 0x0F
        if i % 2 == 0:
            chunk = nib
        else:
            packed.append(chunk | (nib << 4))
    packed.append(chunk)  # odd count: the last low nibble alone
    packed = np.array(packed, np.uint8)
    assert np.array_equal(lh.codes(packed, 4, 255), q + 8)
    a = np.arange(255, dtype=np.float32) * np.float32(0.125)
    got, _ = lh.lm_head_logits(a[None, :], lh.FMT_INT4, packed, np.ones(1, np.float32), 1, 255)
    assert got[0, 0] == float(np.dot(a.astype(np.float64), q.astype(np.float64)))
    # and quantize packs the same way: low nibble first over the global index
    # (-1, 1, 0.25) -> values (-7, 7, 2), codes (1, 15, 10) -> bytes 0xF1, 0x0A
    qq, _ = lh.quantize(np.array([[-1.0, 1.0, 0.25]], np.float32), 1, 3, 4)
    assert qq.tolist() == [0xF1, 0x0A]


@pytest.mark.parametrize("fmt,group", [(lh.FMT_F32, None), (lh.FMT_INT8, None), (lh.FMT_INT8, 4),
                                       (lh.FMT_INT4, None), (lh.FMT_INT4, 2)])
def test_brute_force_tiny_shapes(fmt, group):
    rnd = np.random.default_rng(5)
    B, H, V = 3, 8, 5
    x = rnd.standard_normal((B, H)).astype(np.float32)
    w = rnd.standard_normal((V, H)).astype(np.float32)
    if fmt == lh.FMT_F32:
        data, scales = w.reshape(-1), None
    else:
        data, scales = lh.quantize(w, V, H, fmt, group)
    got, absd = lh.lm_head_logits(x, fmt, data, scales, V, H, group)
    g = group or H
    for b in range(B):
        for v in range(V):
            acc = 0.0
            tot = 0.0
            for h in range(H):
                if fmt == lh.FMT_F32:
                    wv = float(w[v, h])
                else:
                    idx = v * H + h
                    if fmt == lh.FMT_INT8:
                        c = int(data[idx]) - 128
                    else:
                        byte = int(data[idx // 2])
                        c = ((byte >> 4) if idx % 2 else (byte & 15)) - 8
                    wv = c * float(scales[v * (H // g) + h // g])
                acc += float(x[b, h]) * wv
                tot += abs(float(x[b, h]) * wv)
            assert got[b, v] == pytest.approx(acc, rel=1e-12, abs=1e-12)
            assert absd[b, v] == pytest.approx(tot, rel=1e-12)


def test_f32_bound_holds_for_orders_and_catches_slips():
    rnd = np.random.default_rng(11)
    H = 768
    x = rnd.standard_normal(H).astype(np.float32)
    w = (rnd.standard_normal(H) * 0.05).astype(np.float32)
    exact = float(np.dot(x.astype(np.float64), w.astype(np.float64)))
    tot = float(np.abs(x.astype(np.float64) * w.astype(np.float64)).sum())
    bound = lh.f32_bound(tot, H)
    prods = (x * w).astype(np.float32)
    for order in (np.arange(H), np.arange(H)[::-1], rnd.permutation(H)):
        s = np.float32(0.0)
        for i in order:
            s = np.float32(s + prods[i])
        assert abs(float(s) - exact) <= bound
    assert abs(float(prods.reshape(-1, 4).sum(axis=1, dtype=np.float32).sum(dtype=np.float32))
               - exact) <= bound
    # a dropped term or a scale off by one row is far outside the bound
    assert abs((exact - float(prods[7])) - exact) > bound or abs(float(prods[7])) < bound
    assert abs(exact * 1.01 - exact) > bound
