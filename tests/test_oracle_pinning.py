"""Pins the CPU oracle (CPU only, no GPU).

The reference ships no golden vectors for its quantizers or kernels (its tests
only compare end-to-end text), so each oracle function is pinned here by
something independent of its own formula:

* fp16 conversion: numpy's IEEE binary16 conversion, exhaustively;
* Q8_0: hand-derived known-answer blocks (exact codes, round-half-away ties);
* Q4_K / Q6_K: lattice superblocks whose optimal codes are known by
  construction (the search must recover them exactly), decoded by three
  independent restatements of the reference's own decoders;
* error bounds and special cases that any correct quantizer meets.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import quant as Q

RNG = np.random.default_rng(20261201)


# ---------------------------------------------------------------- fp16 --

def test_f16_decode_exhaustive():
    bits = np.arange(65536, dtype=np.uint32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([Q.f16_bits_to_f32(int(b)) for b in bits[::7]], np.float32)
    ref = ref[::7]
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(got[finite], ref[finite])
    assert np.all(np.isnan(got[~finite] * 0) | np.isinf(got[~finite]))


def test_f16_encode_matches_numpy_rne():
    vals = np.concatenate([
        RNG.standard_normal(3000).astype(np.float32) * 10.0 ** RNG.integers(-9, 5, 3000),
        np.float32([0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e-8, 5.96e-8, 2.98e-8, 2.99e-8, -6.1e-5]),
        # exact ties between adjacent fp16 values (RNE must pick the even mantissa)
        (np.float16(1.0).astype(np.float32) + np.float32(2.0 ** -11) * np.arange(1, 9, 2, dtype=np.float32)),
    ]).astype(np.float32)
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([Q.f32_to_f16_bits(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(got, ref)


# ---------------------------------------------------------------- Q8_0 --

def _q8_block(values):
    packed = oracle.quantize_q8_0(np.asarray(values, np.float32).reshape(1, 32))
    d = packed[0, 0:2].view(np.float16)[0]
    q = packed[0, 2:34].view(np.int8)
    return float(d), q.astype(np.int32)


def test_q8_0_known_answers():
    # amax 127 -> d = 1 exactly: integer inputs come back as their own codes
    ints = np.arange(-127, -95, dtype=np.float32)
    ints[5] = 127.0
    d, q = _q8_block(ints)
    assert d == 1.0
    np.testing.assert_array_equal(q, ints.astype(np.int32))
    # round-half-away-from-zero ties (GLSL round_away, vulkan.py:143-148)
    vals = np.zeros(32, np.float32)
    vals[:8] = [127, 0.5, 1.5, -0.5, -1.5, 2.5, -2.5, 126.5]
    d, q = _q8_block(vals)
    assert d == 1.0
    np.testing.assert_array_equal(q[:8], [127, 1, 2, -1, -2, 3, -3, 127])
    # d = 2: codes are x / 2, negative amax maps to -127
    vals = 2.0 * np.arange(-127, -127 + 32 * 8, 8, dtype=np.float32)
    vals = np.clip(vals, -254, 254)
    d, q = _q8_block(vals)
    assert d == 2.0 and q[0] == -127
    np.testing.assert_array_equal(q, np.round(vals / 2).astype(np.int32))
    # all-zero block: d = 0 and codes 0 (inv_scale = 0 branch)
    d, q = _q8_block(np.zeros(32))
    assert d == 0.0 and not q.any()


def test_q8_0_error_bound_and_padding():
    x = (RNG.standard_normal((64, 96)) * RNG.uniform(0.01, 3, (64, 1))).astype(np.float32)
    packed = oracle.quantize_q8_0(x)
    deq = oracle.dequant_q8_0(packed, 96)
    d, q = Q.decode_q8_0_codes(packed)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    d_exact = amax / 127
    bound = d_exact / 2 + 127 * np.abs(d - d_exact) + 1e-7
    err = np.abs(deq.reshape(-1, 32) - x.reshape(-1, 32)).max(axis=1)
    assert np.all(err <= bound)
    assert np.all(np.abs(q).max(axis=1) == 127)
    # K not a multiple of 32 is zero-padded (gguf.py:125-127)
    xp = x[:, :70]
    np.testing.assert_array_equal(oracle.quantize_q8_0(xp), oracle.quantize_q8_0(np.pad(xp, ((0, 0), (0, 26)))))


# ---------------------------------------------------------------- Q4_K --

def _q4k_lattice(seed: int):
    """A superblock whose exact Q4_K encoding is known by construction."""
    rng = np.random.default_rng(seed)
    D, Dm = 2.0 ** -10, 2.0 ** -11
    c = rng.integers(1, 64, 8)
    c[rng.integers(8)] = 63          # max scale code 63 -> d = D exactly
    e = rng.integers(0, 64, 8)
    e[rng.integers(8)] = 63          # max min code 63 -> dmin = Dm exactly
    levels = rng.integers(0, 16, (8, 32))
    levels[:, 0] = 0                 # each sub-block spans 0..15
    levels[:, 1] = 15
    for j in range(8):
        rng.shuffle(levels[j])
    x = (D * c[:, None] * levels - Dm * e[:, None]).astype(np.float32).reshape(256)
    return x, D, Dm, c, e, levels.reshape(256)


@pytest.mark.parametrize("decoder", [Q.decode_q4_k_gemv_style, Q.decode_q4_k_embedding_style,
                                     Q.decode_q4_k_gemm_style])
def test_q4_k_lattice_recovered_exactly(decoder):
    xs, expect = [], []
    for seed in range(12):
        x, D, Dm, c, e, lv = _q4k_lattice(seed)
        xs.append(x)
        expect.append((D, Dm, c, e, lv))
    packed = oracle.quantize_q4_k(np.stack(xs))
    d, dmin, sc, mn, q = decoder(packed)
    for i, (D, Dm, c, e, lv) in enumerate(expect):
        assert d[i] == D and dmin[i] == Dm
        np.testing.assert_array_equal(sc[i], c)
        np.testing.assert_array_equal(mn[i], e)
        np.testing.assert_array_equal(q[i], lv)
    # and the value formula reproduces the lattice exactly
    np.testing.assert_array_equal(oracle.dequant_q4_k(packed, 256), np.stack(xs))


def test_q4_k_decoders_agree_on_random_data():
    x = (RNG.standard_normal((40, 1024)) * RNG.uniform(0.001, 2, (40, 1))).astype(np.float32)
    packed = oracle.quantize_q4_k(x)
    ref = oracle.dequant_q4_k(packed, 1024)
    for decoder in (Q.decode_q4_k_gemv_style, Q.decode_q4_k_embedding_style, Q.decode_q4_k_gemm_style):
        vals = Q.q4_k_values_from_codes(*decoder(packed)).reshape(40, 1024)
        np.testing.assert_array_equal(vals, ref)


def test_q4_k_invariants_and_error():
    x = (RNG.standard_normal((64, 2048)) * 0.02).astype(np.float32)
    packed = oracle.quantize_q4_k(x)
    d, dmin, sc, mn, q = Q.decode_q4_k_embedding_style(packed)
    assert sc.max() <= 63 and mn.max() <= 63 and q.max() <= 15
    assert np.all(sc.max(axis=1) == 63)               # d = max_scale / 63 -> the largest code is 63
    assert np.all(d >= 0) and np.all(dmin >= 0)
    deq = oracle.dequant_q4_k(packed, 2048)
    rel = np.sqrt(np.mean((deq - x) ** 2)) / np.std(x)
    assert rel < 0.09, rel                            # ~4.5 bits/weight on Gaussian data
    # within each sub-block, an in-range element is within half a step (+ fp16 slack)
    step = np.repeat((d[:, None] * sc), 32, axis=1).reshape(64, 2048)
    err = np.abs(deq - x)
    assert np.mean(err <= 0.5 * step + 1e-6) > 0.97


def test_q4_k_special_blocks():
    blocks = np.stack([
        np.zeros(256), np.full(256, -1.25), np.abs(RNG.standard_normal(256)), np.full(256, 0.75),
    ]).astype(np.float32)
    packed = oracle.quantize_q4_k(blocks)
    d, dmin, sc, mn, q = Q.decode_q4_k_gemm_style(packed)
    assert d[0] == 0 and dmin[0] == 0 and not q[0].any()          # zero block
    assert d[1] == 0 and not q[1].any() and mn[1].max() == 63       # constant negative: only the min term
    deq = oracle.dequant_q4_k(packed, 256)
    # non-negative block: the least-squares fit may still pick a small negative min; the fit stays close
    assert np.abs(deq[2] - blocks[2]).max() < 0.6 * float(np.repeat(d[2] * sc[2], 32).max())
    np.testing.assert_allclose(deq[1], -1.25, rtol=2e-3)
    np.testing.assert_allclose(deq[3], 0.75, rtol=2e-3)


# ---------------------------------------------------------------- Q6_K --

def _q6k_lattice(seed: int):
    rng = np.random.default_rng(seed)
    dd = 2.0 ** -8
    c = rng.integers(1, 129, 16)
    c[rng.integers(16)] = 128        # block scale codes -c (the max maps to -128)
    levels = rng.integers(1, 64, (16, 16))
    levels[:, 0] = 0                 # the largest |x| sits at level -32 in every sub-block
    for j in range(16):
        rng.shuffle(levels[j])
    x = (dd * c[:, None] * (levels - 32)).astype(np.float32).reshape(256)
    return x, dd, c, levels.reshape(256)


def test_q6_k_lattice_recovered_exactly():
    xs, expect = [], []
    for seed in range(12):
        x, dd, c, lv = _q6k_lattice(seed)
        xs.append(x)
        expect.append((dd, c, lv))
    packed = oracle.quantize_q6_k(np.stack(xs))
    d, scales, q = Q.decode_q6_k_codes(packed)
    for i, (dd, c, lv) in enumerate(expect):
        assert d[i] == -dd                            # d = 1/inv_scale with inv_scale = -128/max_scale
        np.testing.assert_array_equal(scales[i], -c)
        np.testing.assert_array_equal(q[i], lv - 32)
    np.testing.assert_array_equal(oracle.dequant_q6_k(packed, 256), np.stack(xs))


def test_q6_k_error_and_special():
    x = (RNG.standard_normal((32, 1024)) * 0.05).astype(np.float32)
    packed = oracle.quantize_q6_k(x)
    deq = oracle.dequant_q6_k(packed, 1024)
    assert np.sqrt(np.mean((deq - x) ** 2)) / np.std(x) < 0.025
    d, scales, q = Q.decode_q6_k_codes(packed)
    dv = (d[:, None] * np.repeat(scales, 16, axis=1)) * q
    np.testing.assert_array_equal(dv.reshape(32, 1024).astype(np.float32), deq)
    z = oracle.quantize_q6_k(np.zeros((1, 256), np.float32))
    d, scales, q = Q.decode_q6_k_codes(z)
    assert d[0] == 0 and not scales.any() and not q.any()


def test_quantizers_reject_bad_k():
    with pytest.raises(ValueError):
        oracle.quantize_q4_k(np.zeros((2, 100), np.float32))
    with pytest.raises(ValueError):
        oracle.quantize_q6_k(np.zeros((2, 300), np.float32))
