"""GPU parity of the MXFP4 path (decode, layout, matvec) against the CPU oracle.

Bit-exact: device generators, GGUF repack round trip, reference-table decode.
Tolerance (north star): relative L2 <= 1e-5 for f32-accumulated matvec outputs.
"""
import numpy as np
import pytest

import oracle_lib as O
import ttlab_amd

pytestmark = pytest.mark.gpu
N = 2880
TOL = 1e-5


@pytest.fixture(scope="module")
def dev():
    d = ttlab_amd.Device(0)
    print("device:", d.info(), flush=True)
    yield d
    d.close()


def test_device_generators_match_oracle_bits(dev):
    n = 100003
    buf = dev.alloc(n * 4)
    dev.synth_normal(buf, 0x78000001, 5, n, sigma=0.5, mean=1.0)
    assert np.array_equal(buf.download(np.float32, n).view(np.uint32),
                          O.synth_normal(0x78000001, 5, n, sigma=0.5, mean=1.0).view(np.uint32))
    dev.synth_normal_bf16(buf, 0x77000001, 9, n, 0.02)
    assert np.array_equal(buf.download(np.float32, n).view(np.uint32),
                          O.synth_normal_bf16(0x77000001, 9, n, 0.02).view(np.uint32))
    buf.free()
    nb = 5000
    gb = dev.alloc(nb * 17)
    dev.synth_mxfp4_gguf(gb, 0x77000000, 3, nb, 119, 125, block_offset=12345)
    assert np.array_equal(gb.download(np.uint8, nb * 17), O.synth_mxfp4(0x77000000, 3, nb, 119, 125, 12345))
    gb.free()


def test_upload_download_round_trip(dev):
    rows, experts = 48, 3
    blocks = O.synth_mxfp4(1, 2, rows * 90 * experts, 0, 255)
    t = dev.mxfp4_upload(blocks, rows, N, experts)
    assert np.array_equal(t.download_gguf(), blocks)
    t.free()


def test_synthetic_tensor_is_the_oracle_stream_per_expert(dev):
    rows, experts = 32, 3
    t = dev.mxfp4_synthetic(rows, N, experts, 0x77000000, 100)
    got = t.download_gguf().reshape(experts, -1)
    for e in range(experts):
        assert np.array_equal(got[e], O.synth_mxfp4(0x77000000, 100 + e, rows * 90))
    t.free()


def exhaustive_decode_blocks():
    """16 rows x 90 blocks covering every (scale, code) pair: block b of row r has
    scale (r*90+b) % 256 and its bytes walk all 16 codes in both nibbles."""
    blocks = np.zeros((16 * 90, 17), np.uint8)
    for k in range(16 * 90):
        blocks[k, 0] = k % 256
        for i in range(16):
            blocks[k, 1 + i] = ((i + k) % 16) | (((i + 7 * k + 3) % 16) << 4)
    return blocks.reshape(-1)


def test_dequantize_reference_table_bit_exact(dev):
    blocks = exhaustive_decode_blocks()
    t = dev.mxfp4_upload(blocks, 16, N, 1)
    got = t.dequantize(0, mode=0).reshape(-1)
    expected = O.dequant_mxfp4(blocks)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
    t.free()


def test_matvec_decode_instruction_lane_layout(dev):
    """The gfx950 fp4 conversion used by the matvec yields the reference's values:
    low nibble -> element j, high nibble -> element j+16, scale 2^(e-127).  The
    only bit difference is code 8, which the instruction decodes as -0.0 and the
    reference table as +0.0 (equal as numbers)."""
    blocks = exhaustive_decode_blocks()
    t = dev.mxfp4_upload(blocks, 16, N, 1)
    got = t.dequantize(0, mode=1).reshape(-1)
    expected = O.dequant_mxfp4(blocks)
    codes = np.concatenate([blocks.reshape(-1, 17)[:, 1:] & 15, blocks.reshape(-1, 17)[:, 1:] >> 4], axis=1).ravel()
    same_bits = got.view(np.uint32) == expected.view(np.uint32)
    assert np.all(same_bits | ((codes == 8) & (got == 0) & (expected == 0)))
    assert np.all(np.signbit(got[codes == 8]))
    t.free()


def test_prefill_decode_to_bf16_is_exact(dev):
    """The bf16 conversion with the E8M0 scale folded in (the MFMA kernels' weights)
    gives the reference's values for every code and every scale the MFMA path
    supports (E8M0 1..254), code 8 again as -0.0."""
    blocks = exhaustive_decode_blocks()
    t = dev.mxfp4_upload(blocks, 16, N, 1)
    got = t.dequantize(0, mode=2).reshape(-1)
    expected = O.dequant_mxfp4(blocks)
    b = blocks.reshape(-1, 17)
    codes = np.concatenate([b[:, 1:] & 15, b[:, 1:] >> 4], axis=1).ravel()
    scales = np.repeat(b[:, 0], 32)
    same = (got.view(np.uint32) == expected.view(np.uint32)) | ((codes == 8) & (got == 0) & (expected == 0))
    bad_scales = sorted(set(scales[~same].tolist()))
    print("E8M0 values whose bf16 decode differs from the reference:", bad_scales)
    assert all(e in (0, 255) for e in bad_scales), bad_scales
    t.free()


def test_matvec_reference_kat_1080_25(dev):
    # tests/host_dispatch.cpp:92-107
    expert_bytes = N * 90 * 17
    data = np.zeros(2 * expert_bytes, np.uint8)
    blocks = data[expert_bytes:].reshape(-1, 17)
    blocks[:, 0] = 127
    blocks[:, 1:] = 0x21
    t = dev.mxfp4_upload(data, N, N, 2)
    bias = dev.upload(np.full(2 * N, 0.25, np.float32))
    x = dev.upload(np.full(N, 0.5, np.float32))
    y = dev.alloc(N * 4)
    dev.matvec_mxfp4(t, bias, x, y, 1)
    assert np.all(y.download(np.float32) == np.float32(1080.25))
    for b in (bias, x, y):
        b.free()
    t.free()


@pytest.mark.parametrize("emin,emax", [(119, 125), (0, 2), (100, 140)])
def test_matvec_matches_oracle_config0(dev, emin, emax):
    """Config 0: W = 5760 x 2880 as experts 0 and 1 of {2880, 2880, 2}, x ~ N(0,1)."""
    blocks = O.synth_mxfp4(0x77000000, 0, 2 * N * 90, emin, emax)
    x = O.synth_normal(0x78000000, 0, N)
    bias = O.synth_normal(0x78000000, 1, 2 * N, sigma=0.5)
    if emin < 3:
        # products near 2^-128 would vanish next to an O(1) bias; compare the sums themselves
        bias = np.zeros(2 * N, np.float32)
    t = dev.mxfp4_upload(blocks, N, N, 2)
    xb, bb, yb = dev.upload(x), dev.upload(bias), dev.alloc(N * 4)
    for e in range(2):
        dev.matvec_mxfp4(t, bb, xb, yb, e)
        got = yb.download(np.float32)
        assert np.count_nonzero(got - bias[e * N:(e + 1) * N]) > N // 2
        for body in (O.BODY_DEFAULT, O.BODY_V4):
            ref = O.mxfp4_matvec(blocks, bias, N, N, x, expert=e, body=body)
            err = O.rel_l2(got, ref)
            print(f"expert {e} body {body} rel_l2 {err:.3e}")
            assert err <= TOL
    for b in (xb, bb, yb):
        b.free()
    t.free()


@pytest.mark.parametrize("emin,emax", [(250, 255), (255, 255)])
def test_matvec_overflow_band_matches_oracle(dev, emin, emax):
    """E8M0 250..255 with x ~ N(0, 1): partial sums pass 2^128, and every row mixes +inf
    and -inf terms.  Both reference bodies give NaN in every row (model of the CPU
    result for these inputs); the GPU's positions of NaN and infinity equal theirs.
    (Between these and finite results, e.g. E8M0 240..250, the reference's own two
    bodies disagree row by row on NaN, infinity or a finite value, so no per-row bar
    exists there: test_oracle_compute.test_mxfp4_overflow_band_is_order_dependent.)"""
    blocks = O.synth_mxfp4(0x77000000, 0, N * 90, emin, emax)
    x = O.synth_normal(0x78000000, 0, N)
    zero = np.zeros(N, np.float32)
    t = dev.mxfp4_upload(blocks, N, N, 1)
    assert t.edge_scales
    xb, yb = dev.upload(x), dev.alloc(N * 4)
    dev.matvec_mxfp4(t, None, xb, yb, 0)
    got = yb.download(np.float32)
    for body in (O.BODY_DEFAULT, O.BODY_V4):
        ref = O.mxfp4_matvec(blocks, zero, N, N, x, expert=0, body=body)
        assert np.isnan(ref).all()
        assert np.array_equal(np.isnan(got), np.isnan(ref))
        assert np.array_equal(np.isinf(got), np.isinf(ref))
    for b in (xb, yb):
        b.free()
    t.free()


def test_matvec_top_and_bottom_exponents_match_oracle(dev):
    """The decode matvec takes every E8M0 value exactly, E8M0 0 (2^-127) and 255 (2^127
    per reference integer, tensor.cpp:36-44) included.  x is of order 2^-24 in columns
    0..1439 and of order 1 in columns 1440..2879.  Rows 0..1439 hold E8M0 253..255 with
    codes 0, 1, 8 or 9 (|E2M1| <= 0.5, so products stay finite) in the first 45 blocks;
    rows 1440.. hold E8M0 0..2 with any codes in the last 45 blocks (subnormal products;
    no bias, so they are the whole sum).  Every other block is zero codes at E8M0 127
    (the reference's AVX-512 body scales x first, and 2^127 x would overflow there).
    Relative L2 <= 1e-5 against both reference bodies."""
    rng = np.random.default_rng(3)
    half = N // 2
    blocks = np.zeros((N, 90, 17), np.uint8)
    blocks[:, :, 0] = 127
    blocks[:half, :45, 0] = rng.integers(253, 256, (half, 45))
    codes = rng.choice(np.array([0, 1, 8, 9], np.uint8), (half, 45, 32))
    blocks[:half, :45, 1:] = codes[:, :, :16] | (codes[:, :, 16:] << 4)
    blocks[half:, 45:, 0] = rng.integers(0, 3, (N - half, 45))
    blocks[half:, 45:, 1:] = rng.integers(0, 256, (N - half, 45, 16))
    blocks = blocks.ravel()
    x = np.concatenate([O.synth_normal(5, 0, 1440) * np.float32(2.0 ** -24),
                        O.synth_normal(5, 1, N - 1440)]).astype(np.float32)
    zero = np.zeros(N, np.float32)
    t = dev.mxfp4_upload(blocks, N, N, 1)
    assert t.edge_scales
    xb, yb = dev.upload(x), dev.alloc(N * 4)
    dev.matvec_mxfp4(t, None, xb, yb, 0)
    got = yb.download(np.float32)
    assert np.isfinite(got).all()
    for body in (O.BODY_DEFAULT, O.BODY_V4):
        ref = O.mxfp4_matvec(blocks, zero, N, N, x, expert=0, body=body)
        assert np.isfinite(ref).all()
        for rows in (slice(0, half), slice(half, N)):
            err = O.rel_l2(got[rows], ref[rows])
            print(f"body {body} rows {rows.start}..{rows.stop}: rel_l2 {err:.2e}")
            assert err <= TOL
    for b in (xb, yb):
        b.free()
    t.free()


def test_zero_code_rows_give_the_bias_bit_for_bit(dev):
    """Rows made only of codes 0 and 8 (+0 and -0 in E2M1; the reference's table has +0
    for both) give exactly the bias, as the reference's AVX-512 body does: the gfx950
    conversion's -0 for code 8 never reaches an output, because every sum starts at +0
    and +0 + (-0) is +0."""
    rows = 64
    blocks = np.zeros((rows, 90, 17), np.uint8)
    blocks[:, :, 0] = 127
    blocks[:, :, 1:] = np.random.default_rng(4).choice(np.array([0x00, 0x08, 0x80, 0x88], np.uint8), (rows, 90, 16))
    blocks = blocks.ravel()
    bias = O.synth_normal(6, 0, rows, sigma=2.0)
    bias[:4] = [0.0, -0.0, 1e-30, -1e-30]
    x = O.synth_normal(6, 1, N)
    t = dev.mxfp4_upload(blocks, rows, N, 1)
    bb, xb, yb = dev.upload(bias), dev.upload(x), dev.alloc(rows * 4)
    dev.matvec_mxfp4(t, bb, xb, yb, 0)
    got = yb.download(np.float32)
    ref = O.mxfp4_matvec(blocks, bias, rows, N, x, expert=0, body=O.BODY_V4)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    for b in (bb, xb, yb):
        b.free()
    t.free()


def test_mfma_entry_points_refuse_edge_scales(dev):
    """A tensor with a block of E8M0 0 or 255 is flagged at upload, and the batched MFMA
    entry points (whose bf16 weights cannot hold those scales exactly) refuse it
    instead of computing a different result; ordinary scales are accepted."""
    rows = 192
    base = O.synth_mxfp4(0x77000000, 9, rows * 90)
    x = dev.upload(O.synth_normal(7, 0, 4 * N))
    tokens = dev.upload(np.array([0, 2], np.int32))
    out = dev.alloc(4 * rows * 4)
    ok = dev.mxfp4_upload(base, rows, N, 1)
    assert not ok.edge_scales
    dev.matmul_mxfp4_selected(ok, None, x, N, 4, tokens, 2, out, 0)
    ok.free()
    for e in (0, 255):
        blocks = base.copy()
        blocks[17 * 1000] = e
        t = dev.mxfp4_upload(blocks, rows, N, 1)
        assert t.edge_scales
        with pytest.raises(ttlab_amd.TtlError, match="E8M0 scale 0 or 255"):
            dev.matmul_mxfp4_selected(t, None, x, N, 4, tokens, 2, out, 0)
        t.free()
    syn = dev.mxfp4_synthetic(rows, N, 1, 1, 1, emin=0, emax=3)
    assert syn.edge_scales
    syn.free()
    for b in (x, tokens, out):
        b.free()


def test_f16_exact_flag_at_upload(dev):
    """ttl_mxfp4_f16_exact: 1 when every block with a code of nonzero magnitude has E8M0
    scale 114..140 (every weight a normal f16), the range of the f16 down GEMM; a block of
    zero codes does not count, whatever its scale."""
    rows = 64
    base = O.synth_mxfp4(0x77000000, 10, rows * 90)
    t = dev.mxfp4_upload(base, rows, N, 1)
    assert t.f16_exact
    t.free()
    for e, zero_codes, exact in ((113, False, False), (141, False, False), (114, False, True), (140, False, True),
                                 (113, True, True), (200, True, True)):
        blocks = base.copy()
        blocks[17 * 777] = e
        if zero_codes:
            blocks[17 * 777 + 1:17 * 778] = 0x88 if e == 200 else 0  # +0 and -0 codes
        t = dev.mxfp4_upload(blocks, rows, N, 1)
        assert t.f16_exact == exact, (e, zero_codes)
        assert not t.edge_scales
        t.free()
    for emin, emax, exact in ((114, 140, True), (113, 125, False), (119, 141, False)):
        syn = dev.mxfp4_synthetic(rows, N, 2, 1, 1, emin=emin, emax=emax)
        assert syn.f16_exact == exact, (emin, emax)
        syn.free()


def test_config0_as_one_5760_row_matrix(dev):
    """The {2880, 2880, 2} bytes uploaded as one 5760-row matrix (the bench's config-0
    launch) give bitwise the two experts' rows, and the oracle's values."""
    blocks = O.synth_mxfp4(0x77000000, 0, 2 * N * 90)
    x = O.synth_normal(0x78000000, 0, N)
    one = dev.mxfp4_upload(blocks, 2 * N, N, 1)
    two = dev.mxfp4_upload(blocks, N, N, 2)
    xb, y1, y2 = dev.upload(x), dev.alloc(2 * N * 4), dev.alloc(2 * N * 4)
    ids = dev.upload(np.array([0, 1], np.int32))
    dev.matvec_mxfp4(one, None, xb, y1, 0)
    dev.matvec_mxfp4_experts(two, None, xb, 0, ids, 2, y2)
    a, b = y1.download(np.float32), y2.download(np.float32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    zero = np.zeros(2 * N, np.float32)
    ref = np.concatenate([O.mxfp4_matvec(blocks, zero, N, N, x, expert=e, body=O.BODY_V4) for e in range(2)])
    assert O.rel_l2(a, ref) <= TOL
    for buf in (xb, y1, y2, ids):
        buf.free()
    one.free()
    two.free()


def test_expert_indexed_batch_reads_selected_experts(dev):
    E = 8
    blocks = O.synth_mxfp4(0x77000000, 7, E * N * 90)
    bias = O.synth_normal(3, 3, E * N, sigma=0.1)
    experts = np.array([3, 0, 7, 3], np.int32)
    xs = O.synth_normal(4, 4, 4 * N).reshape(4, N)
    t = dev.mxfp4_upload(blocks, N, N, E)
    bb, xb, eb, yb = dev.upload(bias), dev.upload(xs), dev.upload(experts), dev.alloc(4 * N * 4)
    dev.matvec_mxfp4_experts(t, bb, xb, N, eb, 4, yb)
    got = yb.download(np.float32).reshape(4, N)
    for s in range(4):
        ref = O.mxfp4_matvec(blocks, bias, N, N, xs[s], expert=int(experts[s]), body=O.BODY_V4)
        assert O.rel_l2(got[s], ref) <= TOL
    # shared x (stride 0)
    dev.matvec_mxfp4_experts(t, None, xb, 0, eb, 4, yb)
    got = yb.download(np.float32).reshape(4, N)
    zero = np.zeros(E * N, np.float32)
    for s in range(4):
        ref = O.mxfp4_matvec(blocks, zero, N, N, xs[0], expert=int(experts[s]), body=O.BODY_V4)
        assert O.rel_l2(got[s], ref) <= TOL
    for b in (bb, xb, eb, yb):
        b.free()
    t.free()


def test_out_of_range_expert_gives_nan_not_a_fault(dev):
    t = dev.mxfp4_synthetic(64, N, 2, 1, 1)
    x = dev.upload(np.ones(N, np.float32))
    e = dev.upload(np.array([1, 2, -1], np.int32))
    y = dev.alloc(3 * 64 * 4)
    dev.matvec_mxfp4_experts(t, None, x, 0, e, 3, y)
    out = y.download(np.float32).reshape(3, 64)
    assert np.all(np.isfinite(out[0]))
    assert np.all(np.isnan(out[1])) and np.all(np.isnan(out[2]))
    for b in (x, e, y):
        b.free()
    t.free()


def test_shape_errors_are_reported(dev):
    with pytest.raises(ttlab_amd.TtlError, match="cols must be 2880"):
        dev.mxfp4_synthetic(64, 2048, 1, 1, 1)
    with pytest.raises(ttlab_amd.TtlError, match="multiple of 16"):
        dev.mxfp4_synthetic(40, N, 1, 1, 1)
