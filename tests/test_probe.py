"""Measurement probes: the exchange-latency chain the token kernel's design is
priced with (xp_exchange_chain_timed). GPU only; a probe returns a timing,
so the checks are that it runs to completion on every placement and rejects
shapes it cannot lay out."""
import ctypes as C

import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("producers,stride,l2", [(1, 1, 0), (1, 8, 1), (18, 8, 0), (48, 1, 0)])
def test_gpu_exchange_chain_runs(xp, producers, stride, l2):
    ns = C.c_float()
    xp.call("xp_exchange_chain_timed", producers, 16, stride, l2, None, C.byref(ns))
    # one stage is at least a store and a load through the cache hierarchy,
    # and far below the probe's own timeout
    assert 100.0 < ns.value < 1e6, ns.value


@pytest.mark.parametrize("producers,stages,stride,l2", [
    (0, 16, 1, 0),      # no producers
    (257, 16, 1, 0),    # more than 256 producers
    (33, 16, 8, 0),     # more roles than one XCD's workgroups
    (4, 1, 1, 0),       # a chain needs two stages
    (4, 16, 2, 0),      # stride 1 or 8
    (4, 16, 1, 1),      # L2-kept stores need one XCD
])
def test_gpu_exchange_chain_rejects(xp, producers, stages, stride, l2):
    ns = C.c_float()
    with pytest.raises(xp.XposeError):
        xp.call("xp_exchange_chain_timed", producers, stages, stride, l2, None, C.byref(ns))


@pytest.mark.parametrize("same_xcd,pairs,l2", [(1, 1, 0), (0, 1, 0), (1, 2304, 0), (0, 4096, 0), (1, 32, 1)])
def test_gpu_handoff_pingpong_runs(xp, same_xcd, pairs, l2):
    """The two-workgroup hand-off probe finishes every placement and payload;
    a round trip is two hand-offs, each at least a store and a load through
    the cache hierarchy; a payload of several loads a polling thread takes
    longer than one pair (up to 512 pairs, one load a thread, it need not)."""
    ns, xcc = C.c_float(), C.c_uint32()
    xp.call("xp_handoff_pingpong_timed", same_xcd, pairs, l2, 200, None, C.byref(ns), C.byref(xcc))
    assert 200.0 < ns.value < 1e5, ns.value
    if pairs > 1024:
        one = C.c_float()
        xp.call("xp_handoff_pingpong_timed", same_xcd, 1, l2, 200, None, C.byref(one), C.byref(xcc))
        assert ns.value > one.value, (ns.value, one.value)


def test_gpu_handoff_pingpong_rejects(xp):
    ns, xcc = C.c_float(), C.c_uint32()
    for args in ((1, 0, 0, 10), (1, 4097, 0, 10), (0, 1, 1, 10), (1, 1, 0, 0)):
        with pytest.raises(xp.XposeError):
            xp.call("xp_handoff_pingpong_timed", *args, None, C.byref(ns), C.byref(xcc))


def test_gpu_load_latency(xp):
    """Dependent loads: a footprint past the L2 (64 MiB of 128-byte nodes)
    takes longer per load than one that fits its L1 (16 KiB)."""
    small, big = C.c_float(), C.c_float()
    xp.call("xp_load_latency", 16 << 10, 256, 0, None, C.byref(small))
    xp.call("xp_load_latency", 64 << 20, 128, 1, None, C.byref(big))
    assert 10.0 < small.value < big.value < 1e5, (small.value, big.value)
    with pytest.raises(xp.XposeError):
        xp.call("xp_load_latency", 100, 256, 0, None, C.byref(small))
