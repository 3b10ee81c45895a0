"""Pins the oracle's fp8 e4m3 functions (CPU only).

Checks: torch's float8_e4m3fn cast on every bf16 bit pattern and on exact
mid-points, torch's decode table, the absmax/448 block recipe computed with
torch ops (rows and 128 x 128 blocks, including an all-zero block), and the
fp8 grouped GEMM computed with torch on dequantised operands; plus
invariants that do not depend on torch and planted mistakes they catch.
"""
from __future__ import annotations

import numpy as np

from conftest import load_golden
from oracle import moe_oracle as O


def test_e4m3_cast_matches_torch_on_all_bf16_patterns():
    g = load_golden("fp8_e4m3_convert")
    f = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(O.f32_to_e4m3_bits(f), g["bf16_patterns_e4m3"])


def test_e4m3_cast_ties_and_saturation():
    g = load_golden("fp8_e4m3_convert")
    np.testing.assert_array_equal(O.f32_to_e4m3_bits(g["ties"]), g["ties_e4m3"])
    # mid-point 1 + 1/16 lies between 1.0 (mantissa 000, even) and 1.125: ties to even
    assert O.f32_to_e4m3_bits(np.float32([1.0 + 1 / 16]))[0] == 0x38
    # largest finite value and the NaN code
    assert O.e4m3_bits_to_f32(np.uint8([0x7E]))[0] == 448.0
    assert np.isnan(O.e4m3_bits_to_f32(np.uint8([0x7F]))[0])


def test_e4m3_decode_table_matches_torch():
    g = load_golden("fp8_e4m3_convert")
    np.testing.assert_array_equal(O.E4M3_VALUES, g["decode"])


def test_e4m3_round_trip_of_representable_values():
    finite = np.array([b for b in range(256) if (b & 0x7F) != 0x7F], np.uint8)
    vals = O.e4m3_bits_to_f32(finite)
    back = O.f32_to_e4m3_bits(vals)
    # +0 and -0 both survive; every finite code maps back to itself
    np.testing.assert_array_equal(back, finite)


def test_quantize_rows_matches_torch_recipe():
    g = load_golden("fp8_quant_rows")
    bits, scale = O.quantize_fp8_rows(g["x"])
    np.testing.assert_array_equal(scale, g["scale"])
    np.testing.assert_array_equal(bits, g["bits"])
    assert scale[3, 1] == 0 and not bits[3, 128:256].any()


def test_quantize_blocks_matches_torch_recipe():
    g = load_golden("fp8_quant_blocks")
    bits, scale = O.quantize_fp8_blocks(g["w"])
    np.testing.assert_array_equal(scale, g["scale"])
    np.testing.assert_array_equal(bits, g["bits"])


def test_quantize_invariants():
    rng = np.random.default_rng(3)
    x = O.bf16_round(rng.standard_normal((16, 512)).astype(np.float32) * 3)
    bits, scale = O.quantize_fp8_rows(x)
    q = O.e4m3_bits_to_f32(bits).reshape(16, 4, 128)
    # the block absmax maps to the largest code
    np.testing.assert_array_equal(np.abs(q).max(axis=2), np.full((16, 4), 448.0, np.float32))
    # dequantised values are within half an e4m3 step (relative 2^-4) of the input
    d = O.dequant_rows(bits, scale)
    xb = x.reshape(16, 4, 128)
    step = np.maximum(np.abs(xb), scale[:, :, None] * 2.0 ** -6)  # subnormal floor
    assert np.all(np.abs(d.reshape(16, 4, 128) - xb) <= step * 2.0 ** -4 * 1.0001)


def test_grouped_mm_fp8_matches_torch():
    g = load_golden("fp8_grouped_mm")
    offs = np.cumsum(g["counts"])
    out = O.grouped_mm_fp8(g["xq"], g["sx"], g["wq"], g["sw"], offs)
    assert O.max_rel_err(out, g["out"]) < 1e-5


def test_planted_scale_transpose_is_caught():
    """Using the weight scale of the transposed block (a plausible indexing
    mistake) breaks the torch golden."""
    g = load_golden("fp8_grouped_mm")
    offs = np.cumsum(g["counts"])
    sw = g["sw"].copy()
    sw[:, 0, 1], sw[:, 1, 0] = g["sw"][:, 1, 0], g["sw"][:, 0, 1]
    out = O.grouped_mm_fp8(g["xq"], g["sx"], g["wq"], sw, offs)
    assert O.max_rel_err(out, g["out"]) > 1e-2


def _rms_rel(got, ref):
    d = np.asarray(got, np.float64) - ref
    return float(np.sqrt((d ** 2).mean() / (np.asarray(ref, np.float64) ** 2).mean()))


def test_fp8_layer_tracks_bf16_layer():
    """e4m3 keeps 3 mantissa bits (relative step 2^-3), so on random data the
    fp8 forward sits at ~6% RMS from the bf16 forward; the fp8 path's own
    5e-2 tolerance is against this dequantising oracle, not the bf16 layer.
    A planted mistake (the up-projection rows' block scales swapped with the
    gate rows') moves it far away."""
    rng = np.random.default_rng(11)
    T, D, H, E, K = 64, 256, 128, 4, 2
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    w13 = O.bf16_round((rng.standard_normal((E, 2 * H, D)) * 0.02).astype(np.float32))
    w13[:, H:] *= 8.0  # up rows on a different scale from gate rows
    w2 = O.bf16_round((rng.standard_normal((E, D, H)) * 0.02).astype(np.float32))
    scores, idx = O.router_topk(rng.standard_normal((T, E)).astype(np.float32), K, "softmax", True)
    w13q, s13 = O.quantize_fp8_blocks(w13)
    w2q, s2 = O.quantize_fp8_blocks(w2)
    out8 = O.moe_forward_fp8(x, scores, idx, w13q, s13, w2q, s2, E, False)
    ref = O.moe_forward(x, scores, idx, w13, w2, E, False)
    assert 1e-3 < _rms_rel(out8, ref) < 0.1
    s13_bad = s13[:, ::-1].copy()
    bad = O.moe_forward_fp8(x, scores, idx, w13q, s13_bad, w2q, s2, E, False)
    assert _rms_rel(bad, ref) > 0.5
