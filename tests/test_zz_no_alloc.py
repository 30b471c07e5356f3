"""xp_mv_int4_noalloc, the allocation-free variant of xp_mv_int4 (its partial
sums and tickets in a fixed per-GPU device array): called through the C ABI
and checked against xp_mv_int4 on the same inputs, bit for bit where both
take the same plan, and against the oracle at 1e-5 of max|y| where the fixed
scratch makes it take the split-k plan instead. Calls follow each other on
one stream, a larger then a smaller one, so the second runs on what the
first left in the scratch.
"""
import numpy as np
import pytest

from test_matvec import run_mv, synth_case


def run_na(xp, wq, sc, x, rows, cols, fmt, split=0):
    dw, ds, dx = (xp.DeviceBuffer.from_array(a) for a in (wq, sc, x))
    dout = xp.DeviceBuffer(cols * 4)
    dout.upload(np.full(cols, -1e30, np.float32))      # sentinel: every output written
    xp.call("xp_mv_int4_noalloc", dout.vp, dx.vp, dw.vp, ds.vp, fmt, rows, cols, split, None)
    xp.synchronize()
    return dout.download(np.float32)


def same_bits(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.gpu
def test_gpu_noalloc_matvec_equals_library_entry(xp, xo):
    X = xp
    # 1. a shape deeper than one workgroup's k (16384 x 4096, 512 blocks):
    #    the automatic plan's k-chunk workgroups, whose partials (8 chunks x
    #    64 groups x 64 = 32,768 floats) and arrival tickets are in the fixed
    #    scratch; twice, so the second call runs on tickets the first
    #    returned to zero
    print("case noalloc deep k-chunks 16384 x 4096", flush=True)
    wq, sc, x = synth_case(X, 16384, 4096, seed=5)
    b = run_mv(X, wq, sc, x, 16384, 4096, 0)
    for _ in range(2):
        assert same_bits(run_na(X, wq, sc, x, 16384, 4096, 0), b)
    want = xo.mv_km4(x, wq, sc, 16384, 4096, 0)
    assert np.abs(b - want).max() / np.abs(want).max() < 1e-5
    # down 6912 x 1152, automatic plan: column-slice workgroups over the
    # whole k (no partials, no tickets)
    print("case noalloc down auto", flush=True)
    wq, sc, x = synth_case(X, 6912, 1152)
    a = run_na(X, wq, sc, x, 6912, 1152, 0)
    b = run_mv(X, wq, sc, x, 6912, 1152, 0)
    assert same_bits(a, b)
    # 2. a smaller call right after: q 1152 x 1024 (2 chunks)
    print("case noalloc q auto", flush=True)
    wq, sc, x = synth_case(X, 1152, 1024, seed=7)
    a = run_na(X, wq, sc, x, 1152, 1024, 0)
    assert same_bits(a, run_mv(X, wq, sc, x, 1152, 1024, 0))
    # 3. explicit split-k on the gate shape, twice (second call on the same
    #    scratch, tickets back at zero)
    print("case noalloc gate split 5", flush=True)
    wq, sc, x = synth_case(X, 1152, 6912, seed=9)
    ref = run_mv(X, wq, sc, x, 1152, 6912, 0, 5)
    for _ in range(2):
        assert same_bits(run_na(X, wq, sc, x, 1152, 6912, 0, 5), ref)
    # 4. and smaller again, no partials at all (one workgroup per column group)
    print("case noalloc gate auto", flush=True)
    a = run_na(X, wq, sc, x, 1152, 6912, 0)
    assert same_bits(a, run_mv(X, wq, sc, x, 1152, 6912, 0))
    want = xo.mv_km4(x, wq, sc, 1152, 6912, 0)
    assert np.abs(a - want).max() / np.abs(want).max() < 1e-5


@pytest.mark.gpu
def test_gpu_noalloc_matvec_limits(xp, xo):
    X = xp
    # A shape too deep for column slices (k 16384) whose k-chunk plan needs
    # more partials than the fixed scratch (8 chunks x 600 groups x 64 =
    # 307,200 floats > 262,144): the split-k plan (4 chunks) instead; the
    # library entry keeps the k-chunk plan.
    print("case noalloc fallback 16384 x 38400", flush=True)
    rows, cols = 16384, 38400
    wq, sc, x = synth_case(X, rows, cols, seed=11)
    a = run_na(X, wq, sc, x, rows, cols, 0)
    b = run_mv(X, wq, sc, x, rows, cols, 0)
    want = xo.mv_km4(x, wq, sc, rows, cols, 0)
    m = np.abs(want).max()
    assert not (a == np.float32(-1e30)).any()
    assert np.abs(a - want).max() / m < 1e-5
    assert np.abs(a - b).max() / m < 1e-5
    # An explicit split whose partials do not fit is refused with a message,
    # and the scratch is usable afterwards.
    print("case noalloc refused split", flush=True)
    wq2, sc2, x2 = synth_case(X, 1152, 262144, seed=13)
    with pytest.raises(X.XposeError) as e:
        run_na(X, wq2, sc2, x2, 1152, 262144, 0, 2)
    assert "partial floats" in str(e.value) and "262144" in str(e.value)
    wq3, sc3, x3 = synth_case(X, 6912, 1152, seed=15)
    assert same_bits(run_na(X, wq3, sc3, x3, 6912, 1152, 0), run_mv(X, wq3, sc3, x3, 6912, 1152, 0))
