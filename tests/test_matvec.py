"""int4 KM4 matvec: the oracle pinned against independent references (CPU),
and the gfx950 kernel against the oracle (GPU).

Reference harnesses this follows: examples/llm/matvec_bench.cpp (nib() hash
fixture, -1e30 poisoning, rel < 1e-4 against max|gold|, :45-55, :300-324) and
decode.cpp matvec_selftest (random shapes, err/rms < 1e-4, :2444-2569).
"""
import numpy as np
import pytest

from conftest import allclose_report

# (name, rows = K, cols = N) — matvec_bench.cpp:30-38 and decode.cpp:2466-2470.
SHAPES = [("q", 1152, 1024), ("kv", 1152, 256), ("o_proj", 1024, 1152),
          ("gate", 1152, 6912), ("down", 6912, 1152), ("lm_head_8k", 1152, 8192)]


def dense_from_km4(xo, wq, rows, cols):
    """[rows][cols] int8 weights (nibble - 8) through the oracle's unpack."""
    out = np.empty(rows * cols, np.int8)
    xo.lib().xo_unpack_km4(out, np.ascontiguousarray(wq, np.uint32), rows, cols)
    return out.reshape(rows, cols)


def scales_dense(sc, fmt, rows, cols):
    """[nblk][cols] fp32 scales from any of the three planes."""
    nblk = rows // 32
    if fmt == 2:
        return np.asarray(sc, np.float32).reshape(nblk, cols)
    q = np.asarray(sc, np.uint16).reshape(nblk // 4, cols, 4)
    planes = q.transpose(0, 2, 1).reshape(nblk, cols)
    if fmt == 0:
        return planes.view(np.float16).astype(np.float32)
    return (planes.astype(np.uint32) << 16).view(np.float32)


def synth_case(xp, rows, cols, seed=0x5EED0001, fmt=0):
    wq = xp.synth_nibbles(rows, cols, seed, 1)
    sc16 = xp.synth_scales(rows, cols, seed, 2, 0.02, 0)
    if fmt == 0:
        sc = sc16
    elif fmt == 1:
        # bf16 payload: the fp16 scale's value truncated to bf16 precision.
        f = scales_dense(sc16, 0, rows, cols)
        bits = (f.view(np.uint32) >> 16).astype(np.uint16)
        nblk = rows // 32
        sc = np.ascontiguousarray(bits.reshape(nblk // 4, 4, cols).transpose(0, 2, 1)).ravel()
    else:
        sc = np.ascontiguousarray(scales_dense(sc16, 0, rows, cols)).ravel()
    x = xp.synth_normal(rows, seed, 3)
    return wq, sc, x


# ---------------------------------------------------------------- CPU ----

def test_unpack_closed_form(xo):
    """Every nibble value at every word position decodes to nibble - 8."""
    rows, cols = 32, 64
    wq = np.zeros(rows * cols // 8, np.uint32)
    # Column t, block 0: word c holds nibbles (t + c*8 + i) % 16 at position i.
    for t in range(64):
        for c in range(4):
            w = 0
            for i in range(8):
                w |= ((t + c * 8 + i) % 16) << (4 * i)
            wq[t * 4 + c] = w
    dense = dense_from_km4(xo, wq, rows, cols)
    for t in range(64):
        for k in range(32):
            assert dense[k, t] == ((t + k) % 16) - 8


def test_q4dot8_closed_form(xo):
    """q4dot8 against the explicit sum for all 16 values in all 8 slots."""
    v = np.arange(1, 9, dtype=np.float32) * 0.25
    for n in range(16):
        for slot in range(8):
            w = (8 << (4 * np.arange(8))).sum() & 0xFFFFFFFF      # every slot = 8 -> 0
            w = int(w) & ~(0xF << (4 * slot)) | (n << (4 * slot))
            assert xo.lib().xo_q4dot8(w, v) == np.float32(v[slot] * (n - 8))


@pytest.mark.parametrize("name,rows,cols", [("small", 128, 128), ("q", 1152, 1024),
                                            ("o_proj", 1024, 1152)])
@pytest.mark.parametrize("fmt", [0, 1, 2])
def test_oracle_vs_float64(xh, xo, name, rows, cols, fmt):
    wq, sc, x = synth_case(xh, rows, cols, fmt=fmt)
    W = dense_from_km4(xo, wq, rows, cols).astype(np.float64)
    S = np.repeat(scales_dense(sc, fmt, rows, cols).astype(np.float64), 32, axis=0)
    want = (x.astype(np.float64)[:, None] * W * S).sum(axis=0)
    got = xo.mv_km4(x, wq, sc, rows, cols, fmt)
    rel = np.abs(got - want).max() / np.abs(want).max()
    assert rel < 1e-5, rel


@pytest.mark.parametrize("name,rows,cols", SHAPES)
def test_oracle_km4_equals_col_gold_on_reference_fixture(xo, name, rows, cols):
    """The reference's own cross-layout check: KM4 vs the COL gold on the nib()
    hash, in = sin(0.37 i) * 0.5, scale = 0.02 + 0.001 (i % 7)."""
    nblk = rows // 32
    wk = np.empty(rows * cols // 8, np.uint32)
    wc = np.empty(rows * cols // 8, np.uint32)
    xo.lib().xo_pack_km4_hash(wk, rows, cols)
    xo.lib().xo_pack_col_hash(wc, rows, cols)
    x = (np.sin(np.arange(rows, dtype=np.float64) * 0.37) * 0.5).astype(np.float32)
    s = (np.float32(0.02) + np.float32(0.001) * (np.arange(nblk * cols) % 7).astype(np.float32))
    s = s.astype(np.float32)
    gold = np.empty(cols, np.float32)
    xo.lib().xo_matvec_q4_col(gold, x, wc, s, rows, cols)
    got = xo.mv_km4(x, wk, s, rows, cols, 2)
    assert np.abs(gold).max() > 0
    rel = np.abs(got - gold).max() / np.abs(gold).max()
    assert rel < 1e-4, rel


def test_oracle_split_equals_unsplit(xh, xo):
    rows, cols = 1152, 1024
    wq, sc, x = synth_case(xh, rows, cols, fmt=2)
    full = xo.mv_km4(x, wq, sc, rows, cols, 2)
    for split in (2, 4, 5):
        part = np.empty(split * cols, np.float32)
        xo.lib().xo_mv_km4_split(part, x, wq, sc.ctypes.data, 2, rows, cols, split)
        red = np.empty(cols, np.float32)
        xo.lib().xo_mv_reduce(red, part, cols, split)
        rel = np.abs(red - full).max() / np.abs(full).max()
        assert rel < 1e-5, (split, rel)


# ---------------------------------------------------------------- GPU ----

def run_mv(xp, wq, sc, x, rows, cols, fmt, split=0):
    dw, ds, dx = (xp.DeviceBuffer.from_array(a) for a in (wq, sc, x))
    dout = xp.DeviceBuffer(cols * 4)
    dout.upload(np.full(cols, -1e30, np.float32))      # sentinel: every output written
    xp.call("xp_mv_int4", dout.vp, dx.vp, dw.vp, ds.vp, fmt, rows, cols, split, None)
    xp.synchronize()
    return dout.download(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("name,rows,cols", SHAPES + [("lm_head", 1152, 262144)])
@pytest.mark.parametrize("fmt", [0, 1, 2])
def test_gpu_matvec_matches_oracle(xp, xo, name, rows, cols, fmt):
    print(f"case matvec {name} {rows}x{cols} fmt={fmt}", flush=True)
    wq, sc, x = synth_case(xp, rows, cols, fmt=fmt)
    want = xo.mv_km4(x, wq, sc, rows, cols, fmt)
    got = run_mv(xp, wq, sc, x, rows, cols, fmt)
    assert not (got == np.float32(-1e30)).any(), "outputs left untouched"
    # fp32 accumulation in a different order: 1e-5 of max|y| (north_star bar 1e-3).
    rel = np.abs(got - want).max() / np.abs(want).max()
    assert rel < 1e-5, rel


@pytest.mark.gpu
@pytest.mark.parametrize("split", [1, 2, 3, 5, 9])
def test_gpu_matvec_split_variants(xp, xo, split):
    rows, cols = 1152, 6912
    print(f"case matvec split={split}", flush=True)
    wq, sc, x = synth_case(xp, rows, cols)
    want = xo.mv_km4(x, wq, sc, rows, cols, 0)
    got = run_mv(xp, wq, sc, x, rows, cols, 0, split)
    ok, msg = allclose_report(got, want, 0, 1e-5 * np.abs(want).max())
    assert ok, msg
    # Deterministic: the same call twice gives the same bits.
    again = run_mv(xp, wq, sc, x, rows, cols, 0, split)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


@pytest.mark.gpu
def test_gpu_matvec_reference_fixture(xp, xo):
    """The nib() fixture at the gate shape through the fp32 [b][col] plane."""
    rows, cols = 1152, 6912
    nblk = rows // 32
    wk = np.empty(rows * cols // 8, np.uint32)
    xo.lib().xo_pack_km4_hash(wk, rows, cols)
    x = (np.sin(np.arange(rows, dtype=np.float64) * 0.37) * 0.5).astype(np.float32)
    s = (np.float32(0.02) + np.float32(0.001) * (np.arange(nblk * cols) % 7).astype(np.float32))
    gold = np.empty(cols, np.float32)
    wc = np.empty(rows * cols // 8, np.uint32)
    xo.lib().xo_pack_col_hash(wc, rows, cols)
    xo.lib().xo_matvec_q4_col(gold, x, wc, s.astype(np.float32), rows, cols)
    got = run_mv(xp, wk, s.astype(np.float32), x, rows, cols, 2)
    assert np.abs(got - gold).max() / np.abs(gold).max() < 1e-4


@pytest.mark.gpu
def test_gpu_unpack_bit_exact(xp, xo):
    rows, cols = 1152, 1024
    wq = xp.synth_nibbles(rows, cols, 7, 9)
    dw = xp.DeviceBuffer.from_array(wq)
    dout = xp.DeviceBuffer(rows * cols)
    xp.call("xp_unpack_km4", dout.vp, dw.vp, rows, cols, None)
    xp.synchronize()
    got = dout.download(np.int8)
    want = dense_from_km4(xo, wq, rows, cols).ravel()
    assert np.array_equal(got, want)


@pytest.mark.gpu
def test_gpu_fp16_decode_all_patterns(xp, xo):
    src = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ds = xp.DeviceBuffer.from_array(src)
    dout = xp.DeviceBuffer(65536 * 4)
    xp.call("xp_fp16_decode", dout.vp, ds.vp, 65536, None)
    xp.synchronize()
    got = dout.download(np.float32)
    want = np.array([xo.lib().xo_fp16_to_fp32(int(h)) for h in range(65536)], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name,rows,cols", [("q", 1152, 1024), ("kv", 1152, 256),
                                            ("o_proj", 1024, 1152), ("down", 6912, 1152),
                                            ("gate", 1152, 6912), ("deep", 16384, 4096)])
def test_gpu_matvec_auto_plan_repeatable(xp, xo, name, rows, cols):
    """The automatic plan (split 0): column-slice workgroups over the whole k
    for the Gemma shapes (k <= 8192: no partials, no tickets), and for the
    deep one (k 16384) workgroup tasks per (column group, k-chunk), 8 chunks
    whose last arrival sums the partials in order. The same call twice gives
    the same bits."""
    print(f"case matvec auto plan {name}", flush=True)
    wq, sc, x = synth_case(xp, rows, cols)
    a = run_mv(xp, wq, sc, x, rows, cols, 0)
    b = run_mv(xp, wq, sc, x, rows, cols, 0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    want = xo.mv_km4(x, wq, sc, rows, cols, 0)
    assert np.abs(a - want).max() / np.abs(want).max() < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("cols", [(1024, 256, 256), (6912, 6912)], ids=["qkv", "gate_up"])
def test_gpu_matvec_multi_matches_oracle(xp, xo, cols):
    """xp_mv_int4_multi: matrices of different widths sharing one input (the
    session's q | k | v and gate | up launches), each against the oracle."""
    import ctypes as C
    X = xp
    rows = 1152
    print(f"case matvec multi {cols}", flush=True)
    x = X.synth_normal(rows, 0x5EED0001, 3)
    mats = [(X.synth_nibbles(rows, c, 0x5EED0001, 10 + i),
             X.synth_scales(rows, c, 0x5EED0001, 20 + i, 0.02, 0)) for i, c in enumerate(cols)]
    dx = X.DeviceBuffer.from_array(x)
    dws = [X.DeviceBuffer.from_array(w) for w, _ in mats]
    dss = [X.DeviceBuffer.from_array(s) for _, s in mats]
    douts = [X.DeviceBuffer(c * 4) for c in cols]
    for d, c in zip(douts, cols):
        d.upload(np.full(c, -1e30, np.float32))
    n = len(cols)
    P = C.c_void_p * n
    outs = P(*[d.vp for d in douts])
    wqs = P(*[d.vp for d in dws])
    scs = P(*[d.vp for d in dss])
    cs = (C.c_uint32 * n)(*cols)
    X.call("xp_mv_int4_multi", n, outs, dx.vp, wqs, scs, cs, 0, rows, None)
    X.synchronize()
    for i, c in enumerate(cols):
        got = douts[i].download(np.float32)
        want = xo.mv_km4(x, mats[i][0], mats[i][1], rows, c, 0)
        assert not (got == np.float32(-1e30)).any(), i
        assert np.abs(got - want).max() / np.abs(want).max() < 1e-5, i


@pytest.mark.gpu
def test_gpu_matvec_batch_timed_leaves_the_product(xp, xo):
    """xp_mv_int4_batch_timed (launches captured into one HIP graph, best of
    the replays) computes what xp_mv_int4 computes, bit for bit, on every
    replay: after 4 copies x 3 replays the output equals a single launch's,
    and the reported time is positive; the same-size read in the batch form
    reports a positive time too."""
    import ctypes as C
    rows, cols, copies = 1152, 6912, 4
    print(f"case matvec batch timed {rows}x{cols} x{copies}", flush=True)
    wq, sc, x = synth_case(xp, rows, cols, seed=21)
    want = run_mv(xp, wq, sc, x, rows, cols, 0)
    dws = [xp.DeviceBuffer.from_array(wq) for _ in range(copies)]
    dss = [xp.DeviceBuffer.from_array(sc) for _ in range(copies)]
    dx = xp.DeviceBuffer.from_array(x)
    dout = xp.DeviceBuffer(cols * 4)
    dout.upload(np.full(cols, -1e30, np.float32))
    W = (C.c_void_p * copies)(*[d.ptr for d in dws])
    S = (C.c_void_p * copies)(*[d.ptr for d in dss])
    ms = C.c_float()
    xp.call("xp_mv_int4_batch_timed", dout.vp, dx.vp, W, S, copies, 0, rows, cols, 0, copies, 3, None,
            C.byref(ms))
    xp.synchronize()
    got = dout.download(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert ms.value > 0.0
    ref = xo.mv_km4(x, wq, sc, rows, cols, 0)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5
    nb = 1 << 20
    bufs = [xp.DeviceBuffer(nb) for _ in range(2)]
    for b in bufs:
        xp.call("xp_memset", b.vp, 1, nb)
    P = (C.c_void_p * 2)(*[b.ptr for b in bufs])
    xp.call("xp_stream_read_rot_batch_timed", P, 2, nb, 0, 4, 3, None, C.byref(ms))
    assert ms.value > 0.0
