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
