"""The out-of-process probe plumbing (engine._child_ok, ek_probe) on CPU:
a child that exits cleanly reads as success, anything else as failure."""

from enginekernel_amd import ek_probe
from enginekernel_amd import engine as E


def test_child_probe_plumbing():
    assert E._child_ok(["noop"])
    assert not E._child_ok(["no-such-probe"])
    assert not E._child_ok(["shape", "1"])          # malformed shape arguments
    assert ek_probe.main(["noop"]) == 0 and ek_probe.main([]) == 2
