"""Pins the oracle's format decoders (oracle/ttlab_oracle.c a1/a2).

Known answers are the reference's own (tenstorrent/tt-lab src/tests.cpp:38-52);
the exhaustive checks compare against closed forms computed independently in
numpy (IEEE binary16 widening, E2M1 x 2^(e-127), BF16 round-to-nearest-even).
"""
import numpy as np
import pytest

import oracle_lib as O

lib = O.lib

# OCP MX E2M1 magnitudes for codes 0..7 (sign is bit 3); an independent statement of
# the reference's doubled-integer table (tensor.cpp:34).
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def e2m1(code):
    # the reference's table maps code 8 (E2M1 -0) to integer 0, i.e. +0.0
    v = E2M1[code & 7]
    return -v if (code & 8 and v != 0.0) else v


def test_reference_float_format_kats():
    # src/tests.cpp:38-42
    assert lib.orc_fp16_to_fp32(0x3C00) == 1.0
    assert lib.orc_fp16_to_fp32(0xBC00) == -1.0
    assert lib.orc_fp16_to_fp32(0x0001) == np.ldexp(1.0, -24)
    assert lib.orc_mxfp4_scale(127) == 0.5
    # src/tests.cpp:43-51 (BF16 round to nearest even)
    assert lib.orc_fp32_to_bf16(1.0) == 0x3F80
    assert lib.orc_fp32_to_bf16(1.00390625) == 0x3F80
    assert lib.orc_fp32_to_bf16(np.float32(1.005)) == 0x3F81


def test_fp16_exhaustive_against_numpy():
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = halves.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_fp16_to_fp32(int(h)) for h in halves], np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))


def test_bf16_rounding_against_closed_form():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)
    bits = bits[(bits & 0x7F800000) != 0x7F800000]  # finite inputs
    vals = bits.view(np.float32)
    got = np.array([lib.orc_fp32_to_bf16(float(v)) for v in vals], np.uint16)
    # round to nearest even on the upper 16 bits, written as an integer comparison
    upper = (bits >> 16).astype(np.uint64)
    rem = (bits & 0xFFFF).astype(np.uint64)
    up = (rem > 0x8000) | ((rem == 0x8000) & (upper & 1 == 1))
    expected = (upper + up).astype(np.uint16)
    assert np.array_equal(got, expected)


def test_mxfp4_scale_all_exponents():
    for e in range(256):
        assert lib.orc_mxfp4_scale(e) == np.float32(np.ldexp(1.0, e - 128)), e
    # e = 255 is a finite power of two, never NaN (tensor.cpp:36-44)
    assert np.isfinite(lib.orc_mxfp4_scale(255))


def test_mxfp4_weight_table_exhaustive():
    """All 16 codes x 256 exponents against E2M1 * 2^(e-127) in float64, rounded once."""
    blocks = np.zeros((256, 17), np.uint8)
    blocks[:, 0] = np.arange(256)
    # byte i (i<8) holds code 2i (low) and 2i+1 (high); bytes 8..15 repeat
    for i in range(16):
        lo, hi = (2 * i) % 16, (2 * i + 1) % 16
        blocks[:, 1 + i] = lo | (hi << 4)
    out = O.dequant_mxfp4(blocks.reshape(-1)).reshape(256, 32)
    with np.errstate(over="ignore"):
        for e in range(256):
            for i in range(16):
                lo, hi = (2 * i) % 16, (2 * i + 1) % 16
                exp_lo = np.float32(e2m1(lo) * np.ldexp(1.0, e - 127))
                exp_hi = np.float32(e2m1(hi) * np.ldexp(1.0, e - 127))
                assert out[e, i].tobytes() == exp_lo.tobytes(), (e, lo)
                assert out[e, 16 + i].tobytes() == exp_hi.tobytes(), (e, hi)
    # code 8 is +0.0 (not -0.0)
    assert np.signbit(out[:, [i for i in range(16) if (2 * i) % 16 == 8]]).sum() == 0


def test_mxfp4_element_order_ggml_layout():
    """GGML block_mxfp4: byte j's low nibble is element j, its high nibble element j+16."""
    rng = np.random.default_rng(7)
    block = rng.integers(0, 256, 17, dtype=np.uint8)
    block[0] = 127
    got = O.dequant_mxfp4(block)
    for j in range(16):
        assert got[j] == np.float32(e2m1(block[1 + j] & 15) * 1.0)
        assert got[j + 16] == np.float32(e2m1(block[1 + j] >> 4) * 1.0)


@pytest.mark.parametrize("t,n,expected", [(0, 2880, 11520), (8, 2880, 3060), (39, 2880, 1530),
                                          (30, 64, 128), (8, 33, -1), (39, 31, -1), (2, 32, -1)])
def test_tensor_row_bytes(t, n, expected):
    # tensor.cpp:136-157: MXFP4 row 1530 B at 2880 columns, Q8_0 3060 B
    assert lib.orc_tensor_row_bytes(t, n) == expected


def test_splitmix64_counter_form():
    """orc_hash(seed, 0, i) is output i of Vigna's splitmix64 started at `seed`."""
    def splitmix64(state, count):
        out = []
        m = (1 << 64) - 1
        for _ in range(count):
            state = (state + 0x9E3779B97F4A7C15) & m
            z = state
            z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
            z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
            out.append(z ^ (z >> 31))
        return out
    assert splitmix64(1234567, 1)[0] == 6457827717110365317  # published first output for seed 1234567
    ref = splitmix64(0x77000000, 64)
    assert [lib.orc_hash(0x77000000, 0, i) for i in range(64)] == ref


def test_synthetic_normal_moments_and_exactness():
    x = O.synth_normal(0x78000001, 3, 200000)
    assert abs(float(x.mean())) < 0.01
    assert abs(float(x.var()) - 1.0) < 0.01
    assert float(np.abs(x).max()) < 6.0
    # every value is an integer multiple of 2^-24 (exact integer generation, one rounding)
    k = x.astype(np.float64) * 2**24
    assert np.array_equal(k, np.round(k))
    # slices regenerate identically
    assert np.array_equal(O.synth_normal(0x78000001, 3, 100, offset=500), x[500:600])


def test_synthetic_mxfp4_distribution():
    blocks = O.synth_mxfp4(0x77000000, 1, 50000).reshape(-1, 17)
    scales = blocks[:, 0]
    assert scales.min() == 119 and scales.max() == 125
    counts = np.bincount(scales - 119, minlength=7)
    assert counts.min() > 50000 / 7 * 0.95
    codes = np.concatenate([blocks[:, 1:] & 15, blocks[:, 1:] >> 4]).ravel()
    c16 = np.bincount(codes, minlength=16)
    assert c16.min() > codes.size / 16 * 0.98
    again = O.synth_mxfp4(0x77000000, 1, 10, block_offset=777).reshape(-1, 17)
    assert np.array_equal(again, blocks[777:787])


def test_synthetic_q8_0_and_bf16():
    q = O.synth_q8_0(5, 2, 1000).reshape(-1, 34)
    scales = q[:, :2].copy().view(np.uint16).ravel().view(np.float16).astype(np.float32)
    assert scales.min() >= 2.0**-12 and scales.max() < 2.0**-11
    b = O.synth_bf16(5, 3, 40000)
    exps = (b >> 7) & 0xFF
    assert set(np.unique(exps)) == {120, 121, 122, 123}
    assert np.array_equal(O.synth_bf16(5, 3, 7, offset=1001), b[1001:1008])


# ---- the MXFP8 quantizer of the scaled prefill path (tests/brute_force.py) ----------------

def e4m3_table():
    """Every finite OCP E4M3 value by code (bits S.EEEE.MMM; E = 0 subnormal m x 2^-9;
    S.1111.111 is NaN), enumerated from the definition."""
    vals = {}
    for code in range(256):
        e, m, s = (code >> 3) & 15, code & 7, -1.0 if code & 0x80 else 1.0
        if e == 15 and m == 7:
            continue
        vals[code] = s * (m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
    return vals


def test_e4m3_rounding_against_brute_force_nearest():
    import brute_force as B
    table = e4m3_table()
    codes = np.array(list(table), np.int64)
    values = np.array([table[c] for c in codes])
    assert values.max() == 448.0 and values[values > 0].min() == 2.0 ** -9
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.uniform(-460, 460, 4000), rng.uniform(-0.03, 0.03, 4000),
                        values, (values[:-1] + values[1:]) / 2])  # grid points and neighbours' midpoints
    got = B.e4m3_round(v)
    for x, g in zip(v, got):
        d = np.abs(values - x)
        near = codes[d == d.min()]
        # ties go to the even code (an even mantissa); +0 and -0 are the same value
        best = [c for c in near if c & 1 == 0] or list(near)
        assert g == table[int(best[0])], (x, g)


def test_mxfp8_exponent_rule_brute_force_and_e8m0_floor():
    import brute_force as B
    rng = np.random.default_rng(4)
    m = np.concatenate([np.ldexp(rng.uniform(0.5, 1.0, 3000), rng.integers(-149, 128, 3000)),
                        [448.0, np.nextafter(448.0, 500), 1.75, float(np.nextafter(np.float32(1.75), 2)),
                         2.0 ** -120, 1.5 * 2.0 ** -121, 2.0 ** -126, 1e-40, 1.75 * 2.0 ** -119,
                         float(np.nextafter(np.float32(1.75 * 2.0 ** -119), 1))]]).astype(np.float32)
    blocks = np.zeros((m.size, 32), np.float32)
    blocks[:, 5] = -m
    blocks[:, 6] = m / 3
    X, finite = B.mxfp8_exponents(blocks)
    assert finite.all()
    for mi, xi in zip(m.astype(np.float64), X):
        want = next(k for k in range(-127, 200) if mi / 2.0 ** k <= 448.0)  # the smallest, floor -127
        assert xi == want, (mi, xi, want)
    # maxima at most 448 x 2^-127 = 1.75 x 2^-119 take E8M0 byte 0 (the rule without the floor
    # gives -128..-134 below 1.75 x 2^-120) and stay finite, small and exact where E4M3 holds them
    q = B.mxfp8_dequantize(blocks[-6:-1])
    assert np.all(X[-6:-1] == -127)
    assert np.array_equal(q[:3, 5], blocks[-6:-3, 5])  # 2^-120, 1.5 x 2^-121 and 2^-126 are E4M3 x 2^-127
    assert np.all(np.abs(q[:, 5]) <= np.abs(blocks[-6:-1, 5]) * 1.07)
    assert B.mxfp8_exponents(blocks[-1:])[0][0] == -126
