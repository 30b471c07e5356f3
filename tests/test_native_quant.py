"""Native-format weights (GGUF Q8_0 / Q5_0 / Q4_K / Q6_K, no requantisation):
the repack to slot-interleaved planes and reconstruct() (quant_repack.cpp),
the native-layout dequant and fused matvec (llm_quant.cl:83-322) and the
repacked matvecs, plain and split-k (llm_quant.cl:340-615).

Bars are the reference's own (examples/llm/quant_test.cpp): dequant
bit-exact against the from-spec CPU dequantiser (:290-340), reconstruct() ==
dequant bit for bit (:620-640), every matvec within 1e-5 of max|out| of the
float64 product of the dequantised matrix (:365-405, :690-720), every output
written (sentinel prefill). Inputs follow its random_blocks (:237-259):
random bytes with each fp16 field's exponent rebiased into [8, 22], and a
synthetic case of 130 rows (not a multiple of 64, so the last slot group is
padded) by 128 (1024 for the super-block formats) columns."""
import numpy as np
import pytest

Q8_0, Q5_0, Q4_K, Q6_K = 8, 6, 12, 14
# type: (elements per block, bytes per block, fp16 field offsets, reduction multiple)
FMT = {Q8_0: (32, 34, (0,), 32), Q5_0: (32, 22, (0,), 32), Q4_K: (256, 144, (0, 2), 256),
       Q6_K: (256, 210, (208,), 256)}
NAMES = {Q8_0: "Q8_0", Q5_0: "Q5_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}
SENTINEL = np.float32(-1.0e30)


def random_blocks(t, nblocks, rng):
    """random_blocks of quant_test.cpp:237-259: uniform bytes, each fp16
    field given a sign, a random mantissa and an exponent in [8, 22]."""
    elems, size, fields, _ = FMT[t]
    raw = rng.integers(0, 256, nblocks * size, dtype=np.uint8).reshape(nblocks, size)
    for off in fields:
        h = (rng.integers(0, 2, nblocks) << 15) | rng.integers(0, 1024, nblocks) \
            | ((8 + rng.integers(0, 15, nblocks)) << 10)
        raw[:, off] = (h & 0xFF).astype(np.uint8)
        raw[:, off + 1] = (h >> 8).astype(np.uint8)
    return raw.reshape(-1)


def synth_shape(t):
    return 130, (1024 if FMT[t][0] == 256 else 128)


def case(t, rows, cols, seed):
    rng = np.random.default_rng(seed)
    raw = random_blocks(t, rows * cols // FMT[t][0], rng)
    x = rng.uniform(-1.0, 1.0, cols).astype(np.float32)
    return raw, x


# ---------------------------------------------------------------- CPU ----

def test_rq_layout_sizes_and_refusals(xh):
    X = xh
    l = X.rq_layout(Q6_K, 130, 1024)
    slots = 192 * 32
    assert (l.padded_rows, l.nkb) == (192, 32)
    assert (l.quant_bytes, l.high_bytes, l.scale_bytes, l.bias_bytes) == \
        (slots * 16, slots * 8, slots * 8, 0)
    assert l.native_bytes == 130 * 4 * 210
    l = X.rq_layout(Q8_0, 64, 64)
    assert (l.quant_bytes, l.high_bytes, l.scale_bytes, l.bias_bytes) == (128 * 32, 0, 128 * 4, 0)
    l = X.rq_layout(Q4_K, 1, 256)
    assert (l.padded_rows, l.bias_bytes, l.high_bytes) == (64, 64 * 8 * 4, 0)
    l = X.rq_layout(Q5_0, 64, 32)
    assert (l.high_bytes, l.native_bytes) == (64 * 4, 64 * 22)
    for t, rows, cols in [(Q4_K, 64, 128), (Q6_K, 64, 1000), (Q8_0, 64, 48), (2, 64, 64),
                          (Q8_0, 0, 64)]:
        with pytest.raises(X.XposeError):
            X.rq_layout(t, rows, cols)


@pytest.mark.parametrize("t", [Q8_0, Q5_0, Q4_K, Q6_K], ids=NAMES.get)
def test_rq_repack_matches_oracle_and_reconstructs_dequant(xh, xo, t):
    """The product's planes equal the oracle's (the reference's loops) byte
    for byte, padding included; reconstruct() == dequantize bit for bit on
    both sides (quant_test.cpp:620-640)."""
    X = xh
    rows, cols = synth_shape(t)
    raw, _ = case(t, rows, cols, 11 + t)
    want = X.dequantize(t, raw, rows * cols).reshape(rows, cols)
    assert np.array_equal(want.view(np.uint32),
                          xo.dequantize(t, raw, rows * cols).reshape(rows, cols).view(np.uint32))
    got = X.rq_repack(t, raw, rows, cols, threads=3)
    ref = xo.rq_repack(t, raw, rows, cols)
    for k in ("quant", "high", "scale", "bias"):
        if ref[k] is None:
            assert got[k] is None, k
        else:
            assert np.array_equal(got[k].view(np.uint32), ref[k].view(np.uint32)), k
    rec = X.rq_reconstruct(got)
    assert np.array_equal(rec.view(np.uint32), want.view(np.uint32))
    orec = xo.rq_reconstruct(t, ref, rows, cols)
    assert np.array_equal(orec.view(np.uint32), want.view(np.uint32))
    # the padded slot rows 130..191 hold zero planes
    l = got["layout"]
    sc = got["scale"].reshape(l.padded_rows // 64, l.nkb, 64, -1)
    assert not sc[-1, :, rows % 64:, :].any()


def test_rq_repack_gemma_shapes(xh):
    """At the shapes Gemma-3-1B's Q4_K_M file holds these formats in
    (agent-docs/gguf.md:136-139): reconstruct == dequantize bit for bit."""
    X = xh
    for t, rows, cols in [(Q5_0, 1024, 1152), (Q8_0, 1536, 1152), (Q4_K, 1152, 6912),
                          (Q6_K, 1152, 6912)]:
        raw, _ = case(t, rows, cols, 5)
        want = X.dequantize(t, raw, rows * cols).reshape(rows, cols)
        got = X.rq_repack(t, raw, rows, cols)
        assert np.array_equal(X.rq_reconstruct(got).view(np.uint32), want.view(np.uint32)), t


# ---------------------------------------------------------------- GPU ----

def dev_out(xp, n):
    d = xp.DeviceBuffer(n * 4)
    d.upload(np.full(n, SENTINEL, np.float32))
    return d


def check_mv(got, want, what):
    assert not (got == SENTINEL).any(), f"{what}: outputs left untouched"
    rel = np.abs(got.astype(np.float64) - want).max() / np.abs(want).max()
    assert rel < 1e-5, (what, rel)


@pytest.mark.gpu
@pytest.mark.parametrize("t", [Q8_0, Q5_0, Q4_K, Q6_K], ids=NAMES.get)
def test_gpu_dequant_native_bit_exact(xp, t):
    X = xp
    rows, cols = synth_shape(t)
    print(f"case dequant_native {NAMES[t]} {rows}x{cols}", flush=True)
    raw, _ = case(t, rows, cols, 21 + t)
    n = rows * cols
    want = X.dequantize(t, raw, n)
    dsrc = X.DeviceBuffer.from_array(raw)
    dout = dev_out(X, n)
    X.call("xp_dequant_native", dout.vp, dsrc.vp, t, n, None)
    X.synchronize()
    got = dout.download(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("t", [Q8_0, Q5_0, Q4_K, Q6_K], ids=NAMES.get)
def test_gpu_mv_native(xp, t):
    X = xp
    for rows, cols in [synth_shape(t), (1152, 6912 if FMT[t][0] == 256 else 1152)]:
        print(f"case mv_native {NAMES[t]} {rows}x{cols}", flush=True)
        raw, x = case(t, rows, cols, 31 + t)
        w = X.dequantize(t, raw, rows * cols).reshape(rows, cols).astype(np.float64)
        want = w @ x.astype(np.float64)
        dsrc, dx = X.DeviceBuffer.from_array(raw), X.DeviceBuffer.from_array(x)
        dout = dev_out(X, rows)
        X.call("xp_mv_native", dout.vp, dx.vp, dsrc.vp, t, rows, cols, None)
        X.synchronize()
        check_mv(dout.download(np.float32), want, f"mv_native {NAMES[t]} {rows}x{cols}")


# Gemma-3-1B shapes per format (outputs x reduction): Q5_0 / Q8_0 hold the
# 1152-wide matrices, Q4_K / Q6_K the 6912-wide ffn_down and attn_output.
GEMMA = {Q5_0: [(6912, 1152), (1024, 1152)], Q8_0: [(6912, 1152), (256, 1152)],
         Q4_K: [(1152, 6912), (1152, 1024)], Q6_K: [(1152, 6912), (1152, 1024)]}
# Wide, shallow shapes (>= 64 row groups, <= 40 k-blocks): with split 0 the
# launcher runs one workgroup per row group (Q5_0 / Q8_0 6912 x 1152 above).
WIDE = {Q4_K: [(4096, 1024)], Q6_K: [(4096, 1024)]}


@pytest.mark.gpu
@pytest.mark.parametrize("t", [Q8_0, Q5_0, Q4_K, Q6_K], ids=NAMES.get)
def test_gpu_mv_rq(xp, t):
    """Plain (split 1), split-k (4) and the launcher's choice (0) against the
    float64 product; each call repeated gives the same bits."""
    X = xp
    shapes = [synth_shape(t)] + [s for s in GEMMA[t] + WIDE.get(t, []) if s[1] % FMT[t][3] == 0]
    for rows, cols in shapes:
        raw, x = case(t, rows, cols, 41 + t)
        w = X.dequantize(t, raw, rows * cols).reshape(rows, cols).astype(np.float64)
        want = w @ x.astype(np.float64)
        planes = X.rq_repack(t, raw, rows, cols)
        dw = X.RqWeights(planes)
        dx = X.DeviceBuffer.from_array(x)
        for split in (1, 4, 0):
            print(f"case mv_rq {NAMES[t]} {rows}x{cols} split={split}", flush=True)
            dout = dev_out(X, rows)
            X.call("xp_mv_rq", dout.vp, dx.vp, X.C.byref(dw.tensor), split, None)
            X.synchronize()
            got = dout.download(np.float32)
            check_mv(got, want, f"mv_rq {NAMES[t]} {rows}x{cols} split={split}")
            X.call("xp_mv_rq", dout.vp, dx.vp, X.C.byref(dw.tensor), split, None)
            X.synchronize()
            assert np.array_equal(dout.download(np.float32).view(np.uint32), got.view(np.uint32))
        dw.close()


@pytest.mark.gpu
def test_gpu_mv_rq_rejects_bad_arguments(xp):
    X = xp
    planes = X.rq_repack(Q5_0, case(Q5_0, 64, 64, 1)[0], 64, 64)
    dw = X.RqWeights(planes)
    dx = X.DeviceBuffer.from_array(np.zeros(64, np.float32))
    dout = X.DeviceBuffer(64 * 4)
    t = X.RqTensor.from_buffer_copy(dw.tensor)
    t.high = None
    with pytest.raises(X.XposeError):
        X.call("xp_mv_rq", dout.vp, dx.vp, X.C.byref(t), 0, None)
    t = X.RqTensor.from_buffer_copy(dw.tensor)
    t.cols = 48
    with pytest.raises(X.XposeError):
        X.call("xp_mv_rq", dout.vp, dx.vp, X.C.byref(t), 0, None)
    with pytest.raises(X.XposeError):
        X.call("xp_mv_rq", dx.vp, dx.vp, X.C.byref(dw.tensor), 0, None)
    dw.close()
