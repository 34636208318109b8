"""Synthetic gpt-oss MoE layers for the parity tests.

Host copies come from the oracle's generators; device copies from the product's
device generators (the two are pinned bit-equal by test_gpu_mxfp4.py).
"""
import ctypes as C

import numpy as np

import oracle_lib as O

N = 2880
W_SEED = 0x77000001
X_SEED = 0x78000001
GATE_STREAM, UP_STREAM, DOWN_STREAM = 1000, 2000, 3000
ROUTER_STREAM, BIAS_STREAM = 20, 30


class HostLayer:
    """Host copy of a synthetic MoE layer.  fill_experts (optional) limits the expert
    matrices generated to those experts; the others stay zero (for oracle runs that
    only read the listed experts)."""

    def __init__(self, experts=32, used=4, biases=False, seed=W_SEED, fill_experts=None, scales=None):
        """scales: optional {"gate"|"up"|"down": (emin, emax)} E8M0 ranges (default 119..125)."""
        self.experts, self.used, self.seed = experts, used, seed
        self.scales = {k: (119, 125) for k in ("gate", "up", "down")}
        self.scales.update(scales or {})
        self.router_w = O.synth_normal_bf16(seed, ROUTER_STREAM, experts * N, 0.02)
        if biases:
            self.router_b = O.synth_normal(seed, BIAS_STREAM, experts, sigma=0.1)
            self.gate_b = O.synth_normal(seed, BIAS_STREAM + 1, experts * N, sigma=0.5)
            self.up_b = O.synth_normal(seed, BIAS_STREAM + 2, experts * N, sigma=0.5)
            self.down_b = O.synth_normal(seed, BIAS_STREAM + 3, experts * N, sigma=0.5)
        else:
            self.router_b = np.zeros(experts, np.float32)
            self.gate_b = np.zeros(experts * N, np.float32)
            self.up_b = np.zeros(experts * N, np.float32)
            self.down_b = np.zeros(experts * N, np.float32)
        per = N * 90 * 17
        fill = range(experts) if fill_experts is None else sorted(set(int(e) for e in fill_experts))
        for name, stream in (("gate", GATE_STREAM), ("up", UP_STREAM), ("down", DOWN_STREAM)):
            arr = np.zeros(experts * per, np.uint8)
            for e in fill:
                arr[e * per:(e + 1) * per] = O.synth_mxfp4(seed, stream + e, N * 90, *self.scales[name])
            setattr(self, name, arr)

    def oracle_struct(self):
        s = O.MoeLayer()
        s.hidden, s.expert_hidden, s.experts, s.used = N, N, self.experts, self.used
        s.router_weight = self.router_w.ctypes.data
        s.router_bias = self.router_b.ctypes.data
        s.gate_weight = self.gate.ctypes.data
        s.gate_bias = self.gate_b.ctypes.data
        s.up_weight = self.up.ctypes.data
        s.up_bias = self.up_b.ctypes.data
        s.down_weight = self.down.ctypes.data
        s.down_bias = self.down_b.ctypes.data
        return s

    def oracle_moe(self, x, body):
        out = np.empty(N, np.float32)
        logits = np.empty(self.experts, np.float32)
        idx = np.empty(self.used, np.int64)
        w = np.empty(self.used, np.float32)
        s = self.oracle_struct()
        O.lib.orc_moe(C.byref(s), np.ascontiguousarray(x, np.float32), out, body, logits.ctypes.data,
                      idx.ctypes.data, w.ctypes.data)
        return out, logits, idx, w


class DeviceLayer:
    def __init__(self, dev, host):
        import ttlab_amd
        self.dev, self.host = dev, host
        E = host.experts
        self.gate = dev.mxfp4_synthetic(N, N, E, host.seed, GATE_STREAM, *host.scales["gate"])
        self.up = dev.mxfp4_synthetic(N, N, E, host.seed, UP_STREAM, *host.scales["up"])
        self.down = dev.mxfp4_synthetic(N, N, E, host.seed, DOWN_STREAM, *host.scales["down"])
        self.bufs = [dev.upload(a) for a in (host.router_w, host.router_b, host.gate_b, host.up_b, host.down_b)]
        d = ttlab_amd.MoeLayerDesc()
        d.hidden, d.expert_hidden, d.experts, d.used = N, N, E, host.used
        d.router_weight, d.router_bias, d.gate_bias, d.up_bias, d.down_bias = [b.ptr for b in self.bufs]
        d.gate, d.up, d.down = self.gate.handle, self.up.handle, self.down.handle
        self.desc = d

    def free(self):
        for b in self.bufs:
            b.free()
        for t in (self.gate, self.up, self.down):
            t.free()
