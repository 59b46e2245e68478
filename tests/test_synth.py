"""The synthetic-input generator (synth.py; its GPU twin is checked in test_gpu_parity.py)."""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np

from conftest import synth_module

synth = synth_module()


def scalar_reference(seed: int, stream_id: int, i: int) -> float:
    """The generator spec evaluated with Python integers and the math module, one element at a time."""
    key = synth.stream_key(seed, stream_id)
    z = synth._mix64_int(key + (i + 1) * 0x9E3779B97F4A7C15)
    u1 = ((z >> 32) + 0.5) * 2.0**-32
    u2 = ((z & 0xFFFFFFFF) + 0.5) * 2.0**-32
    return math.sqrt(-2.0 * math.log(u1)) * math.cos(6.283185307179586 * u2)


def f16_rne_exact(v: float) -> int:
    """Round a binary64 value to binary16 (nearest, ties to even) with exact rational arithmetic."""
    if v == 0:
        return 0x8000 if math.copysign(1, v) < 0 else 0
    sign = 0x8000 if v < 0 else 0
    a = Fraction(abs(v))
    # exponent bucket 2^e <= a < 2^(e+1), clamped at the subnormal range (ulp 2^-24 below 2^-14)
    e = max(-14, math.floor(math.log2(a)))
    while e > -14 and Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (e - 10)
    q, r = divmod(a, ulp)
    q = int(q)
    if r > ulp / 2 or (r == ulp / 2 and q % 2 == 1):
        q += 1
    val = q * ulp
    if val >= 65520:
        return sign | 0x7C00
    return sign | int(np.float16(float(val)).view(np.uint16))  # val is representable: exact conversion


def test_known_answers():
    a = synth.normal_f16(42, 3, 8, 0.02).view(np.uint16)
    assert [hex(v) for v in a] == ['0x2713', '0xa441', '0x9cad', '0x2756', '0x1cc9', '0x26a1', '0x1e1d', '0x2660']
    b = synth.normal_f16(7, 1, 8, 1.0).view(np.uint16)
    assert [hex(v) for v in b] == ['0x4051', '0x3a8d', '0x407a', '0x3959', '0x34f3', '0xb7b6', '0x3d81', '0xbdb2']


def test_vectorised_matches_scalar_spec():
    v = synth.normal_f64(123, 2, 1000, 64)
    ref = np.array([scalar_reference(123, 2, 1000 + i) for i in range(64)])
    np.testing.assert_allclose(v, ref, rtol=4e-16, atol=0)


def test_slices_are_independent_of_chunking():
    whole = synth.normal_f16(5, 3, 10000, 0.1)
    pieces = synth.normal_f16(5, 3, 10000, 0.1, chunk=777)
    assert np.array_equal(whole.view(np.uint16), pieces.view(np.uint16))
    np.testing.assert_array_equal(synth.normal_f64(5, 3, 4000, 100), synth.normal_f64(5, 3, 0, 4100)[4000:])


def test_fp16_rounding_is_single_step_nearest_even():
    rng = np.random.default_rng(0)
    vals = list(rng.standard_normal(300) * 3) + [1 + 2**-11, 1 + 3 * 2**-11, 2**-24 * 1.5, 2**-25, 65519.0, 65520.0,
                                                  -(1 + 2**-11 + 2**-40), 0.000061035156249999]
    with np.errstate(over="ignore"):  # 65520 rounds to inf, which is the point of that case
        got = np.array(vals, np.float64).astype(np.float16).view(np.uint16)
    for v, g in zip(vals, got):
        assert int(g) == f16_rne_exact(v), v


def test_distribution_moments():
    x = synth.normal_f64(1, 1, 0, 1 << 18)
    assert abs(x.mean()) < 0.01
    assert abs(x.std() - 1.0) < 0.01
    kurt = ((x - x.mean()) ** 4).mean() / x.var() ** 2
    assert abs(kurt - 3.0) < 0.05


def test_expert_weight_sigmas_by_block():
    cfg = synth.MoeConfig(4, 32, 2, 1, 64)
    ew = synth.gen_expert_weights(cfg, 3).astype(np.float64)
    I, H = cfg.I, cfg.H
    gu = ew[:, : 2 * I].ravel()
    dn = ew[:, 2 * I:].ravel()
    assert abs(gu.std() * math.sqrt(H) - 1) < 0.05
    assert abs(dn.std() * math.sqrt(I) - 1) < 0.05
    raw = synth.normal_f64(3, synth.STREAM_EXPERT_WEIGHTS, 0, ew.size).reshape(ew.shape)
    exp = np.concatenate([raw[:, : 2 * I] / math.sqrt(H), raw[:, 2 * I:] / math.sqrt(I)], axis=1)
    assert np.array_equal(ew.astype(np.float16).view(np.uint16), exp.astype(np.float16).view(np.uint16))


def test_zipf_gate_skews_routing_columns():
    z = synth.zipf_column_scale(64)
    assert abs(z.mean() - 1) < 1e-12 and np.all(np.diff(z) < 0)
    assert z[0] / z[-1] == np.float64(64**1.1)
    cfg = synth.MoeConfig(8, 128, 64, 6, 32, zipf=True)
    wg = synth.gen_w_gate(cfg, 9).astype(np.float64)
    assert wg[:, :4].std() > 3 * wg[:, -16:].std()
