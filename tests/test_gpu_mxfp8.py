"""The scaled path: MXFP4 weights x MXFP8 activations on v_mfma_scale_f32_16x16x128_f8f6f4.

- ttl_mxfp8_dequantize gives bit for bit the host quantizer's values
  (tests/brute_force.mxfp8_dequantize: the rule of TTL_DTYPE_F32_AS_MXFP8).
- The selected-token matmul on the scaled path against the oracle's
  matmul_add_mxfp4_selected_transposed (tensor.cpp:306-495) fed the same dequantized
  activations, and against float64: every product is exact, but the instruction's
  accumulation is not exact in f32.  The measured difference is reported and held to
  1e-5 (per-token relative L2 against the oracle, and |err| / sum |w x| per output
  against float64; measured 7.9e-6 and 2.9e-6, the oracle's own f32 sums 1.5e-7).
- The instruction's own accumulation, pinned by known answers: products aligned to
  the 32-element block's largest, bits below 2^-13 of it dropped; f32 across blocks.
- Benchmark config 2 (512 tokens, 32 experts) on the scaled path stage by stage:
  gate/up + SwiGLU against the host quantizer on the oracle's values, down against
  the oracle fed the device's own MXFP8 hidden, the combine bit for bit.
- moe_batch's experts on the scaled path (activations and the SwiGLU hidden in MXFP8)
  against the oracle on the original activations: the error of the format, reported.
"""
import ctypes as C

import numpy as np
import pytest

import brute_force as B
import oracle_lib as O
import ttlab_amd

pytestmark = pytest.mark.gpu
N = 2880


@pytest.fixture(scope="module")
def dev():
    d = ttlab_amd.Device(0)
    yield d
    d.close()


def test_dequantize_matches_host_quantizer(dev):
    rng = np.random.default_rng(11)
    rows = 8
    x = rng.standard_normal((rows, N)).astype(np.float32)
    # block magnitudes from 2^-30 to 2^30, a zero block, an f32-subnormal block, a block
    # whose maximum sits just above and just below 1.75 x 2^k, a NaN and an inf block
    x.reshape(-1, 32)[:] *= np.float32(2.0) ** rng.integers(-30, 31, (rows * 90, 1)).astype(np.float32)
    blocks = x.reshape(-1, 32)
    blocks[3] = 0.0
    blocks[4] = np.float32(1e-40) * np.arange(32, dtype=np.float32)
    blocks[5, 0] = np.float32(1.75)
    blocks[5, 1:] = 0.1
    blocks[6, 0] = np.nextafter(np.float32(1.75), np.float32(2.0))
    blocks[7, 3] = np.nan
    blocks[8, 9] = np.inf
    # maxima 2^-120, 1.5 x 2^-121 and 2^-126: below 448 x 2^-127, so E8M0 byte 0
    # (without the floor their exponents would wrap to bytes 255, 254 and 249)
    for b, top in ((9, 2.0 ** -120), (10, 1.5 * 2.0 ** -121), (11, 2.0 ** -126)):
        blocks[b] = np.float32(top) * np.linspace(-1, 1, 32, dtype=np.float32)
    expected = B.mxfp8_dequantize(x)
    xb, out = dev.upload(x), dev.alloc(x.nbytes)
    dev.mxfp8_dequantize(xb, ttlab_amd.TTL_DTYPE_F32, rows, out)
    got = out.download(np.float32).reshape(rows, N)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)) or \
        np.array_equal(np.isnan(got), np.isnan(expected)) and np.array_equal(got[~np.isnan(got)], expected[~np.isnan(expected)])
    bits = ttlab_amd.bf16_bits(x)
    bb = dev.upload(bits)
    dev.mxfp8_dequantize(bb, ttlab_amd.TTL_DTYPE_BF16, rows, out)
    got16 = out.download(np.float32).reshape(rows, N)
    exp16 = B.mxfp8_dequantize((bits.astype(np.uint32) << 16).view(np.float32))
    nan = np.isnan(exp16)
    assert np.array_equal(np.isnan(got16), nan) and np.array_equal(got16[~nan], exp16[~nan])
    for b in (xb, out, bb):
        b.free()


def selected(dev, blocks, bias, x, tokens, rows, count, mxfp8):
    t = dev.mxfp4_upload(blocks, rows, N, 1)
    xb, tb = dev.upload(x), dev.upload(np.asarray(tokens, np.int32))
    out = dev.alloc(x.shape[0] * rows * 4)
    dev.fill(out, 0)
    bb = dev.upload(bias) if bias is not None else None
    dev.matmul_mxfp4_selected(t, bb, xb, N, x.shape[0], tb, count, out, 0, mxfp8=mxfp8)
    got = out.download(np.float32).reshape(x.shape[0], rows)
    for b in (xb, tb, out) + ((bb,) if bb else ()):
        b.free()
    t.free()
    return got


@pytest.mark.parametrize("count", [5, 64, 70])
def test_selected_matmul_mxfp8_against_dequantized_oracle(dev, count):
    rows, tokens_total = 192, 80
    blocks = O.synth_mxfp4(0x77000000, 21, rows * 90)
    bias = O.synth_normal(22, 0, rows, sigma=0.1)
    x = O.synth_normal(23, 0, tokens_total * N).reshape(tokens_total, N)
    x.reshape(-1, 32)[:] *= np.float32(2.0) ** np.random.default_rng(4).integers(-3, 4, (tokens_total * 90, 1)).astype(
        np.float32)
    # three blocks of each token at the bottom of the E8M0 range (maxima 2^-120,
    # 1.5 x 2^-121, 2^-126): about zero, never NaN or huge
    for j, top in enumerate((2.0 ** -120, 1.5 * 2.0 ** -121, 2.0 ** -126)):
        x[:, 32 * (7 + 30 * j):32 * (8 + 30 * j)] = np.float32(top) * np.linspace(-1, 1, 32, dtype=np.float32)
    tokens = np.random.default_rng(5).permutation(tokens_total)[:count]
    got = selected(dev, blocks, bias, x, tokens, rows, count, True)
    xq = B.mxfp8_dequantize(x)
    # the oracle (tensor.cpp:306-495, default body) on the dequantized activations
    sel = np.ascontiguousarray(tokens.astype(np.uintp))
    transposed = np.empty(N * count, np.float32)
    O.lib.orc_transpose_selected(N, np.ascontiguousarray(xq.ravel()), sel, count, transposed)
    ref = np.full(tokens_total * rows, np.nan, np.float32)
    ws = np.empty(4 * count + 8, np.float32)
    O.lib.orc_matmul_add_mxfp4_selected_transposed(blocks, bias, rows, N, transposed, sel, count, ref, ws, 0,
                                                   O.BODY_DEFAULT)
    ref = ref.reshape(tokens_total, rows)
    W = B.mxfp4_dense(blocks, rows, N)
    exact = xq[tokens].astype(np.float64) @ W.T + bias
    scale = np.abs(xq[tokens].astype(np.float64)) @ np.abs(W.T)
    err_mx = np.abs(got[tokens] - exact) / scale
    err_ref = np.abs(ref[tokens] - exact) / scale
    rel = max(O.rel_l2(got[t], ref[t]) for t in tokens)
    print(f"count {count}: scaled MFMA |err|/sum|wx| max {err_mx.max():.2e}, oracle f32 {err_ref.max():.2e}; "
          f"worst per-token rel L2 vs the oracle {rel:.2e}")
    assert err_mx.max() <= 1e-5
    assert rel <= 1e-5
    untouched = np.setdiff1d(np.arange(tokens_total), tokens)
    assert not got[untouched].any()


def test_selected_matmul_mxfp8_known_answer(dev):
    """tests/host_dispatch.cpp:108-126 on the scaled path: weights 0x21 at E8M0 127 are
    exact in MXFP4 and x = k/2 (k = 1..16) in MXFP8 (E4M3 holds 3 fraction bits, so 8.5
    would not be); every product is k/2 x 0.5 or k/2 x 1.  Seventeen tokens cross a
    16-token tile."""
    count = 17
    expert_bytes = N * 90 * 17
    data = np.zeros(expert_bytes, np.uint8)
    blocks = data.reshape(-1, 17)
    blocks[:, 0] = 127
    blocks[:, 1:] = 0x21
    rows = N
    x = np.zeros((count + 1, N), np.float32)
    tokens = np.array([count - s for s in range(count)])
    k = [s % 16 + 1 for s in range(count)]
    for s in range(count):
        x[count - s] = k[s] * 0.5
    assert np.array_equal(B.mxfp8_dequantize(x), x)
    got = selected(dev, data, np.full(rows, 0.25, np.float32), x, tokens, rows, count, True)
    for s in range(count):
        assert np.all(got[count - s] == np.float32(1080.0 * k[s] + 0.25)), s
    assert not got[0].any()


def test_scaled_instruction_truncates_within_a_block(dev):
    """The accumulation of v_mfma_scale_f32_16x16x128_f8f6f4, through the selected
    matmul with every weight 1.0 (so each output is the sum of the token's MXFP8
    values): the products of one 32-element block are aligned to the block's largest
    and bits below 2^-13 of it are dropped (256 + 2^-5 is kept, 256 + 2^-6 gives
    256, though f32 holds 256.015625), while block sums are added to each other and
    to the accumulator in f32 (1 + 2^-22 from two blocks is exact).  This is the
    instruction's, not the kernel's: it bounds how closely the scaled path can follow
    the f32 sums of the same MXFP8 values."""
    rows, count = 192, 4
    data = np.zeros(rows * 90 * 17, np.uint8).reshape(-1, 17)
    data[:, 0] = 127
    data[:, 1:] = 0x22  # E2M1 1.0 in both nibbles
    x = np.zeros((count, N), np.float32)
    x[0, 0], x[0, 1] = 256.0, 2.0 ** -5
    x[1, 0], x[1, 1] = 256.0, 2.0 ** -6
    x[2, 0], x[2, 32] = 1.0, 2.0 ** -22
    x[3, 0], x[3, 31] = 1.0, 2.0 ** -12
    assert np.array_equal(B.mxfp8_dequantize(x), x)
    got = selected(dev, data.ravel(), np.zeros(rows, np.float32), x, np.arange(count), rows, count, True)
    assert np.all(got == got[:, :1])
    want = [256.03125, 256.0, 1.0 + 2.0 ** -22, 1.0 + 2.0 ** -12]
    assert [float(v) for v in got[:, 0]] == want, got[:, 0]
    assert float(np.float32(256.0) + np.float32(2.0 ** -6)) == 256.015625  # f32 would hold it


def test_moe_prefill_experts_mxfp8_error_of_the_format(dev):
    """moe_batch's experts (model.cpp:378-460) with bf16 activations: the scaled path
    against the oracle on the same bf16 activations, and the bf16 path's error beside
    it; the scaled path's error is that of MXFP8 activations and hidden."""
    from moe_fixtures import DeviceLayer, HostLayer
    experts, used, count = 8, 4, 96
    host = HostLayer(experts, used, biases=True, seed=0x77000600)
    layer = DeviceLayer(dev, host)
    x = O.synth_normal_bf16(0x78000600, 0, count * N, 1.0).reshape(count, N)
    idx, w = ttlab_amd.balanced_routing(count, experts, used, 7)
    xb = dev.upload(ttlab_amd.bf16_bits(x))
    ib, wb = dev.upload(idx), dev.upload(w)
    ref = np.empty(count * N, np.float32)
    s = host.oracle_struct()
    O.lib.orc_moe_batch_experts(C.byref(s), np.ascontiguousarray(x.ravel()), count,
                                np.ascontiguousarray(idx.astype(np.int64).ravel()), np.ascontiguousarray(w.ravel()), ref,
                                O.BODY_V4)
    ref = ref.reshape(count, N)
    errs = {}
    for name, dtype in (("bf16", ttlab_amd.TTL_DTYPE_BF16), ("mxfp8", ttlab_amd.TTL_DTYPE_BF16_AS_MXFP8)):
        ws = dev.alloc(dev.moe_prefill_workspace_bytes(count, experts, used, dtype))
        out = dev.alloc(count * N * 4)
        dev.moe_prefill_experts(layer.desc, xb, dtype, count, ib, wb, out, ws)
        got = out.download(np.float32).reshape(count, N)
        errs[name] = max(O.rel_l2(got[p], ref[p]) for p in range(count))
        ws.free()
        out.free()
    print(f"moe_batch experts vs the oracle, worst per-token rel L2: bf16 path {errs['bf16']:.2e}, "
          f"scaled MXFP8 path {errs['mxfp8']:.2e}")
    assert errs["bf16"] <= 1e-5
    assert errs["mxfp8"] <= 0.1
    for b in (xb, ib, wb):
        b.free()
    layer.free()


def _block_grid_ok(dev_values, ref, slack, X):
    """True where the device's E4M3 value (x 2^X) is the round-to-nearest-even of some
    value within `slack` of the oracle's pre-rounding `ref` (rounding is monotone, so
    those are the grid points between the roundings of ref - slack and ref + slack),
    and whether it is not the rounding of ref itself."""
    lo = B.e4m3_round(np.ldexp(ref - slack, -X)) * 2.0 ** X
    hi = B.e4m3_round(np.ldexp(ref + slack, -X)) * 2.0 ** X
    mid = B.e4m3_round(np.ldexp(ref, -X)) * 2.0 ** X
    d = dev_values.astype(np.float64)
    return (d >= lo) & (d <= hi), d != mid


def _abs_matvec(blocks, expert, v):
    """sum_k |W[expert][r][k]| |v[k]| per row r, through the oracle's matvec on the
    blocks with every code's sign bit cleared (f32 sums of non-negative terms)."""
    per = N * 90 * 17
    a = np.ascontiguousarray(blocks[expert * per:(expert + 1) * per]).reshape(-1, 17).copy()
    a[:, 1:] &= 0x77
    return O.mxfp4_matvec(a.ravel(), np.zeros(N, np.float32), N, N, np.abs(v).astype(np.float32),
                          body=O.BODY_DEFAULT).astype(np.float64)


def test_moe_prefill_mxfp8_config2_shape_stage_by_stage(dev):
    """Benchmark config 2 on the scaled path (512 bf16 tokens, 32 experts, balanced
    top-4, with biases), each stage against the oracle fed the values the device
    multiplies, on a sample of tokens (moe_batch, model.cpp:378-460):

    - gate/up + SwiGLU: the device's MXFP8 hidden against the host quantizer applied
      to orc_swiglu(orc gate, orc up) on the dequantized MXFP8 activations.  The
      device's gate and up come from the scaled instruction, whose accumulation
      differs from the oracle's f32 sums by up to GU_ERR x sum|w x| (measured 2.9e-6),
      and its SwiGLU uses the hardware exponential and reciprocal (SWIGLU_REL of |h|).
      Propagated through the SwiGLU that gives a bound `slack` per element; an E8M0
      exponent may differ only where a threshold 448 x 2^k lies within the block
      maximum's slack, and an element may differ from the oracle's rounding only to a
      grid point that some value within its slack rounds to.  Those cases are counted.
    - down: the device's down rows against orc_matmul_add_mxfp4_selected_transposed
      (tensor.cpp:319-495, the reference's batched body) fed the device's own
      dequantized hidden: |err| <= 1e-5 sum|w h| per output (the oracle's own f32
      sums are within about 1e-7 of that scale; measured 5.3e-6) and relative L2 <=
      3e-5 per pair (measured 1.6e-5 to 1.9e-5).  The relative L2 cannot reach 1e-5
      on this instruction: it drops product bits below 2^-13 of each 32-element
      block's largest product (test_scaled_instruction_truncates_within_a_block), and
      about a third of the hidden's E4M3 values are that far below their block's
      maximum.  The random activations of the selected matmul, with a narrower range
      per block, stay under 1e-5.
    - combine: the device's output bit for bit against the sum of the device's down
      rows in ascending expert order, each weighted, from +0, unfused
      (model.cpp:450-459).
    """
    from moe_fixtures import DeviceLayer, HostLayer
    GU_ERR, SWIGLU_REL = 2e-5, 4e-6
    count, experts, used = 512, 32, 4
    idx, w = ttlab_amd.balanced_routing(count, experts, used, 11)
    sample = np.random.RandomState(12).choice(count, 6, replace=False)
    host = HostLayer(experts, used, biases=True, seed=0x77000102, fill_experts=idx[sample].ravel())
    layer = DeviceLayer(dev, host)
    dtype = ttlab_amd.TTL_DTYPE_BF16_AS_MXFP8
    bits = ttlab_amd.bf16_bits(O.synth_normal_bf16(0x78000102, 0, count * N, 1.0)).reshape(count, N)
    x = (bits.astype(np.uint32) << 16).view(np.float32)
    bufs = [dev.upload(bits), dev.upload(idx), dev.upload(w)]
    xb, ib, wb = bufs
    ws = dev.alloc(dev.moe_prefill_workspace_bytes(count, experts, used, dtype))
    out = dev.alloc(count * N * 4)
    hid, dwn, scl = dev.alloc(count * used * N * 4), dev.alloc(count * used * N * 4), dev.alloc(count * used * 90)
    bufs += [ws, out, hid, dwn, scl]
    try:
        dev.moe_prefill_experts(layer.desc, xb, dtype, count, ib, wb, out, ws)
        dev.moe_prefill_intermediates(layer.desc, dtype, count, ws, hid, dwn, scl)
        got = out.download(np.float32).reshape(count, N)
        hidden = hid.download(np.float32).reshape(count, used, N)
        down = dwn.download(np.float32).reshape(count, used, N)
        scales = scl.download(np.uint8).reshape(count, used, 90)
        assert np.all(np.isfinite(got)) and np.all(np.isfinite(hidden)) and np.all(np.isfinite(down))

        # gate/up + SwiGLU, pair by pair
        xq = B.mxfp8_dequantize(x[sample]).astype(np.float32)
        exp_moved = elem_moved = elems = 0
        for j, p in enumerate(sample):
            for r in range(used):
                e = int(idx[p, r])
                gate = O.mxfp4_matvec(host.gate, host.gate_b, N, N, xq[j], expert=e, body=O.BODY_DEFAULT)
                up = O.mxfp4_matvec(host.up, host.up_b, N, N, xq[j], expert=e, body=O.BODY_DEFAULT)
                h_ref = np.empty(N, np.float32)
                O.lib.orc_swiglu(gate, up, N, h_ref)
                dg = GU_ERR * _abs_matvec(host.gate, e, xq[j])
                du = GU_ERR * _abs_matvec(host.up, e, xq[j])
                g = np.minimum(gate.astype(np.float64), 7.0)
                y = np.clip(up.astype(np.float64), -7.0, 7.0)
                sg = g / (1.0 + np.exp(-1.702 * g))
                h64 = h_ref.astype(np.float64)
                # |dh/dg| <= 1.2 |y + 1| (x sigma(1.702 x) has slope below 1.1), |dh/du| <= |x sigma|
                slack = 1.2 * (np.abs(y + 1.0) + du) * dg + (np.abs(sg) + 1.2 * dg) * du + SWIGLU_REL * np.abs(h64)
                X_ref, _ = B.mxfp8_exponents(h_ref)
                X_dev = scales[p, r].astype(np.int64) - 127
                blk = h64.reshape(90, 32)
                m_ref = np.abs(blk).max(axis=1)
                m_slack = slack.reshape(90, 32).max(axis=1)
                lo_X, _ = B.mxfp8_exponents(np.repeat(np.maximum(m_ref - m_slack, 0.0), 32).astype(np.float32))
                hi_X, _ = B.mxfp8_exponents(np.repeat(m_ref + m_slack, 32).astype(np.float32))
                assert np.all((X_dev >= lo_X) & (X_dev <= hi_X)), (p, r, np.nonzero(X_dev != X_ref))
                exp_moved += int(np.count_nonzero(X_dev != X_ref))
                Xe = np.repeat(X_dev, 32)
                ok, moved = _block_grid_ok(hidden[p, r], h64, slack, Xe)
                assert ok.all(), (p, r, np.nonzero(~ok)[0][:8])
                elem_moved += int(np.count_nonzero(moved & (np.repeat(X_dev == X_ref, 32))))
                elems += N
        print(f"config 2 scaled gate/up: {elems} hidden values of {len(sample) * used} pairs; E8M0 exponents "
              f"moved by the accumulation: {exp_moved} blocks; E4M3 values one grid point off the oracle's "
              f"rounding, within their bound: {elem_moved}")
        assert elem_moved <= elems // 100

        # down, per expert as moe_batch runs it, on the device's own hidden
        pairs = [(p, r) for p in sample for r in range(used)]
        H = np.ascontiguousarray(np.stack([hidden[p, r] for p, r in pairs]), np.float32)
        ref = np.full(len(pairs) * N, np.nan, np.float32)
        for e in sorted(set(int(idx[p, r]) for p, r in pairs)):
            sel = np.array([k for k, (p, r) in enumerate(pairs) if idx[p, r] == e], np.uintp)
            transposed = np.empty(N * sel.size, np.float32)
            O.lib.orc_transpose_selected(N, H.ravel(), sel, sel.size, transposed)
            wsp = np.empty(4 * sel.size + 8, np.float32)
            O.lib.orc_matmul_add_mxfp4_selected_transposed(host.down, host.down_b, N, N, transposed, sel, sel.size,
                                                           ref, wsp, e, O.BODY_DEFAULT)
        ref = ref.reshape(len(pairs), N)
        worst_rel = worst_abs = 0.0
        for k, (p, r) in enumerate(pairs):
            scale = _abs_matvec(host.down, int(idx[p, r]), H[k])
            worst_abs = max(worst_abs, float((np.abs(down[p, r].astype(np.float64) - ref[k]) / scale).max()))
            worst_rel = max(worst_rel, O.rel_l2(down[p, r], ref[k]))
        print(f"config 2 scaled down vs the oracle on the device's hidden: worst rel L2 {worst_rel:.2e}, "
              f"worst |err| / sum|w h| {worst_abs:.2e}")
        assert worst_abs <= 1e-5
        assert worst_rel <= 3e-5

        # combine: ascending expert order, products rounded, from +0
        for p in sample:
            acc = np.zeros(N, np.float32)
            for r in np.argsort(idx[p], kind="stable"):
                acc = acc + np.float32(w[p, r]) * down[p, r]
            assert np.array_equal(acc.view(np.uint32), got[p].view(np.uint32)), p

        # the error of the format, for the record: the whole layer against the oracle on
        # the unquantized bf16 activations
        full = np.empty(len(sample) * N, np.float32)
        s = host.oracle_struct()
        O.lib.orc_moe_batch_experts(C.byref(s), np.ascontiguousarray(x[sample].ravel()), len(sample),
                                    np.ascontiguousarray(idx[sample].astype(np.int64).ravel()),
                                    np.ascontiguousarray(w[sample].ravel()), full, O.BODY_V4)
        fmt = max(O.rel_l2(got[p], full[j * N:(j + 1) * N]) for j, p in enumerate(sample))
        print(f"config 2 scaled layer vs the oracle on bf16 activations (the MXFP8 format's error): {fmt:.2e}")
    finally:
        for b in bufs:
            b.free()
        layer.free()
