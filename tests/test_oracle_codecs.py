"""Oracle codecs and generators, pinned against the reference's own C++
(qwen3/model.cpp:497-508 compiled in place into oracle/_ref) and numpy."""
import ctypes
import os

import numpy as np
import pytest

import oracle_lib as orc

REF_SO = os.path.join(orc.REF_DIR, "libqwen3_model.so")


def ref_lib():
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (reference sources absent)")
    L = ctypes.CDLL(REF_SO)
    to_bf16 = getattr(L, "_ZN5qwen313float_to_bf16Ef")
    to_bf16.restype, to_bf16.argtypes = ctypes.c_uint16, [ctypes.c_float]
    to_f32 = getattr(L, "_ZN5qwen313bf16_to_floatEt")
    to_f32.restype, to_f32.argtypes = ctypes.c_float, [ctypes.c_uint16]
    return to_bf16, to_f32


def test_bf16_decode_all_codes_match_reference_model_cpp():
    _, to_f32 = ref_lib()
    codes = np.arange(65536, dtype=np.uint16)
    ours = orc.decode(codes, 0)
    for c in range(0, 65536, 7):
        ref = np.float32(to_f32(int(c)))
        if np.isnan(ref):  # ctypes returns NaNs quietened; compare NaN-ness only
            assert np.isnan(ours[c]), hex(c)
            continue
        assert ref.view(np.uint32) == ours[c].view(np.uint32), hex(c)
    # closed form: bf16 is the upper half of the float32 word
    assert np.array_equal(ours.view(np.uint32), codes.astype(np.uint32) << 16)


def test_bf16_encode_matches_reference_model_cpp():
    to_bf16, _ = ref_lib()
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    # include ties (low half exactly 0x8000) and near-ties
    bits[:2000] = (bits[:2000] & 0xFFFF0000) | 0x8000
    bits[2000:3000] = (bits[2000:3000] & 0xFFFF0000) | 0x7FFF
    vals = bits.view(np.float32)
    finite = np.isfinite(vals)
    ours = orc.encode(vals[finite], 0)
    for v, o in zip(vals[finite][:6000], ours[:6000]):
        assert to_bf16(float(v)) == o


def test_bf16_encode_is_round_to_nearest_even():
    # independent closed form: RNE on the float32 bit pattern
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 0x7F7F0000, size=200000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    lo = bits & 0xFFFF
    up = bits >> 16
    expect = up + ((lo > 0x8000) | ((lo == 0x8000) & (up & 1 == 1)))
    assert np.array_equal(orc.encode(vals, 0), expect.astype(np.uint16))


def test_fp16_decode_all_codes_match_numpy():
    codes = np.arange(65536, dtype=np.uint16)
    ours = orc.decode(codes, 1)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp16_encode_matches_numpy_rne_for_normals():
    rng = np.random.default_rng(11)
    vals = (rng.standard_normal(200000) * rng.choice([1e-3, 1.0, 100.0, 3e4], 200000)).astype(np.float32)
    normal = (np.abs(vals) >= 2.0**-14) & (np.abs(vals) < 65504)
    ours = orc.encode(vals[normal], 1)
    ref = vals[normal].astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_fp16_encode_round_trips_every_finite_code():
    codes = np.arange(65536, dtype=np.uint16)
    vals = codes.view(np.float16).astype(np.float32)
    finite = np.isfinite(vals)
    assert np.array_equal(orc.encode(vals[finite], 1), codes[finite])


def test_fp16_overflow_and_nan_become_inf_like_peak_l0():
    # level_zero/peak_l0.cpp:753-759: exponent >= 31 -> signed infinity
    v = np.array([70000.0, -1e9, np.inf, np.nan], np.float32)
    out = orc.encode(v, 1)
    assert list(out[:3]) == [0x7C00, 0xFC00, 0x7C00]
    assert out[3] & 0x7C00 == 0x7C00


def test_uniform_generator_range_moments_and_determinism():
    a = orc.uniform(1 << 20, 1, 0)
    b = orc.uniform(1 << 20, 1, 0)
    c = orc.uniform(1 << 20, 2, 0)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    f = orc.decode(a, 0)
    assert f.min() >= -1.0 and f.max() <= 1.0
    assert abs(f.mean()) < 5e-3 and abs(f.var() - 1 / 3) < 5e-3
    # irregular: no repeating period in the first 1M values
    assert len(np.unique(a)) > 200


def test_uniform_generator_closed_form():
    # element i = (2u - 2^24) / 2^24 with u the top 24 bits of the hash
    L = orc.lib()
    vals = orc.decode(orc.uniform(1000, 42, 1), 1)
    for i in range(0, 1000, 37):
        u = L.orc_hash(42, i) >> 40
        expect = np.float32((2 * u - (1 << 24)) / float(1 << 24)).astype(np.float16).astype(np.float32)
        assert vals[i] == expect


def test_reference_hash_inputs_closed_form():
    # gemv.cpp:91-103
    a, x = orc.reference_gemv_inputs(4, 64, 64, 0)
    fa = orc.decode(a, 0)
    fx = orc.decode(x, 0)
    # bf16 rounding can lift the top of each range to its end point
    assert fa.min() >= 0.25 and fa.max() <= 0.5 and fx.min() >= 0.5 and fx.max() <= 0.75

    def h(i):
        b = i & 0xFFFFFFFF
        b ^= b >> 16
        b = (b * 0x7FEB352D) & 0xFFFFFFFF
        b ^= b >> 15
        b = (b * 0x846CA68B) & 0xFFFFFFFF
        b ^= b >> 16
        return b

    for i in (0, 1, 65, 200, 255):
        expect = np.float32(0.25 + (h(i) & 255) / 1024.0)
        assert a[i] == orc.encode(np.array([expect]), 0)[0]
    for c in (0, 3, 63):
        expect = np.float32(0.5 + (((c * 747796405) & 0xFFFFFFFF) >> 16 & 127) / 512.0)
        assert x[c] == orc.encode(np.array([expect]), 0)[0]
