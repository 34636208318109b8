"""The measurement behind one kernel per dependency level in the decode step
(ttl_measure_handoff): 2880 floats from 180 producer workgroups to 32 consumers that
each need all of them, across a kernel boundary and inside one kernel (agent-scope
release and acquire fences, bounded polling).  Both forms must deliver every value;
the times are printed, not asserted (they vary from box to box)."""
import pytest

import ttlab_amd

pytestmark = pytest.mark.gpu


def test_handoff_across_a_boundary_and_inside_a_kernel():
    dev = ttlab_amd.Device(0)
    try:
        boundary, wrong_b = dev.measure_handoff(0, 50)
        inside, wrong_i = dev.measure_handoff(1, 50)
    finally:
        dev.close()
    print(f"handoff of 2880 floats, 180 producers -> 32 consumers: kernel boundary {boundary:.2f} us, "
          f"inside one kernel (release/acquire fences, flags) {inside:.2f} us")
    assert wrong_b == 0
    assert wrong_i == 0
