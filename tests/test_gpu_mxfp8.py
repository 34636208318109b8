"""The scaled path: MXFP4 weights x MXFP8 activations on v_mfma_scale_f32_16x16x128_f8f6f4.

- ttl_mxfp8_dequantize gives bit for bit the host quantizer's values
  (tests/brute_force.mxfp8_dequantize: the rule of TTL_DTYPE_F32_AS_MXFP8).
- The selected-token matmul on the scaled path against the oracle's
  matmul_add_mxfp4_selected_transposed (tensor.cpp:306-495) fed the same dequantized
  activations, and against float64: every product is exact, but the instruction's
  accumulation is not exact in f32.  The measured difference is reported and held to
  1e-5 (per-token relative L2 against the oracle, and |err| / sum |w x| per output
  against float64; measured 7.9e-6 and 2.9e-6, the oracle's own f32 sums 1.5e-7).
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
