"""The measurements behind one kernel per dependency level in the decode step:

- ttl_measure_handoff: 2880 floats from 180 producer workgroups to 32 consumers that
  each need all of them, across a kernel boundary and inside one kernel (agent-scope
  release and acquire fences, or none: agent-scope stores and loads past the L2s;
  bounded polling); every form must deliver every value.  The fence-free form is the
  cheapest here, where the producers do nothing else; merged into the step's own
  launches (the O projection with the router rows, gate/up with down) it did not gain;
- ttl_measure_boundary: the fixed cost of a kernel boundary in a replayed graph;
- ttl_stream_read / ttl_stream_read_plain: non-temporal against ordinary loads on a
  stream beyond every cache.
The times are printed, not asserted (they vary from box to box)."""
import pytest

import ttlab_amd

pytestmark = pytest.mark.gpu


def test_handoff_across_a_boundary_and_inside_a_kernel():
    dev = ttlab_amd.Device(0)
    try:
        boundary, wrong_b = dev.measure_handoff(0, 50)
        inside, wrong_i = dev.measure_handoff(1, 50)
        nofence, wrong_n = dev.measure_handoff(2, 50)
    finally:
        dev.close()
    print(f"handoff of 2880 floats, 180 producers -> 32 consumers: kernel boundary {boundary:.2f} us, "
          f"inside one kernel (release/acquire fences, flags) {inside:.2f} us, "
          f"inside one kernel without fences (write-through stores, coherent loads) {nofence:.2f} us")
    assert wrong_b == 0
    assert wrong_i == 0
    assert wrong_n == 0


def test_kernel_boundary_cost_is_independent_of_the_grid():
    """ttl_measure_boundary: chains of 200 dependent kernels, each reading in every
    workgroup a word the previous kernel wrote; the time per launch is the boundary's
    fixed cost.  One workgroup of 64 threads and 2880 of 256 must both keep the chain's
    count; the times are printed, not asserted."""
    dev = ttlab_amd.Device(0)
    try:
        small, wrong_s = dev.measure_boundary(200, 1, 64)
        large, wrong_l = dev.measure_boundary(200, 2880, 256)
    finally:
        dev.close()
    print(f"kernel boundary in a replayed graph: {small:.2f} us per launch (1 x 64 threads), "
          f"{large:.2f} us (2880 x 256)")
    assert wrong_s == 0 and wrong_l == 0


def test_nontemporal_and_ordinary_streaming_reads():
    """The weight streams' non-temporal loads against ordinary loads: plain reads of two
    alternating 1.16 GB buffers (beyond every cache), timed per launch; printed."""
    dev = ttlab_amd.Device(0)
    try:
        n = 1158266880  # the bf16 unembedding's bytes
        bufs = [dev.alloc(n) for _ in range(2)]
        for b in bufs:
            dev.fill(b, 0x5a)
        nt = dev.time_stream_read(bufs, n, nontemporal=True, reps=5)
        plain = dev.time_stream_read(bufs, n, nontemporal=False, reps=5)
        for b in bufs:
            b.free()
    finally:
        dev.close()
    print(f"read of {n / 1e9:.2f} GB: non-temporal {nt:.1f} us ({n / nt / 1e3:.0f} GB/s), "
          f"ordinary {plain:.1f} us ({n / plain / 1e3:.0f} GB/s)")
    assert nt > 0 and plain > 0
