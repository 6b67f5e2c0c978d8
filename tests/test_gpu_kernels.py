"""Per-kernel parity of the HIP kernels against the CPU oracle, through the C ABI.

Bar: bit-exact for every output (int32 block dots, f32 GEMV rows, RMSNorm, quantized
activations, RoPE, f16 KV rows, attention, argmax, expf).  Mirrors the reference's
per-kernel GPU tests (src/cuda_resident/tests.rs:765 quantize, :991 argmax, :1028 attention,
:1515 rope split-half, :1445 per-head RMSNorm).
"""
import ctypes as C
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dev(a):
    from camelid_amd.engine import DeviceBuffer
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _buf(nbytes):
    from camelid_amd.engine import DeviceBuffer
    return DeviceBuffer(nbytes)


def _ok(rc):
    from camelid_amd._native import check
    check(rc)


def _repack(native, wire, rows, k):
    from camelid_amd._native import ptr
    q = np.empty(rows * k, np.int8)
    d = np.empty(rows * k // 32, np.uint16)
    _ok(native.camelid_q8_0_repack(ptr(wire, C.c_uint8), rows, k, 34, ptr(q, C.c_int8), ptr(d, C.c_uint16)))
    return q, d


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_expf_device_all_inputs(native, orc):
    """Device expf == glibc expf on every one of the 2^32 f32 bit patterns."""
    chunk = 1 << 27
    xb = _buf(chunk * 4)
    yb = _buf(chunk * 4)
    for start in range(0, 1 << 32, chunk):
        x = np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32).view(np.float32)
        xb.upload(x)
        _ok(native.camelid_hip_expf(xb.ptr, yb.ptr, chunk, None))
        got = yb.download(np.float32, chunk)
        want = orc.expf(x)
        diff = got.view(np.uint32) != want.view(np.uint32)
        diff &= ~(np.isnan(got) & np.isnan(want))
        assert not diff.any(), f"chunk {start:#x}: {np.count_nonzero(diff)} mismatches"


@pytest.mark.parametrize("rows,k", [(2048, 2048), (5632, 2048), (2048, 5632), (1000, 3072), (3072, 8192),
                                    (37, 96), (33, 14336),
                                    # the isolated sweep's two widest shapes: two rows per
                                    # wave (k_gemv_k<K, 2>, rows >= 16384), the lm_head shapes of C1 and C3
                                    (32000, 2048), (128256, 3072), (16385, 4096)])
def test_q8_gemv_bit_exact(native, orc, rows, k):
    from camelid_amd.model import synth_q8_0
    rng = np.random.default_rng(rows * 7 + k)
    # N(0, 0.02) weights as Q8_0 wire blocks (the seeded multi-threaded generator: the widest
    # shapes hold 394M values)
    wire = synth_q8_0(f"gemv{rows}x{k}", 2, rows, k, 0.02)
    q, d = _repack(native, wire, rows, k)
    xs, xq = orc.quantize_q8_0(rng.normal(0, 1, k).astype(np.float32))
    resid = rng.normal(0, 1, rows).astype(np.float32)
    wq, wd, dxq, dxs, dres = _dev(q), _dev(d), _dev(xq), _dev(xs), _dev(resid)
    y = _buf(rows * 4)
    _ok(native.camelid_hip_q8_0_gemv(wq.ptr, wd.ptr, rows, k, dxq.ptr, dxs.ptr, y.ptr, None, None))
    want = orc.q8_0_gemv(wire, rows, k, xs, xq)
    assert np.array_equal(_bits(y.download(np.float32, rows)), _bits(want))
    # fused residual, in place (y aliases resid), as the O / down projections run
    _ok(native.camelid_hip_q8_0_gemv(wq.ptr, wd.ptr, rows, k, dxq.ptr, dxs.ptr, dres.ptr, dres.ptr, None))
    assert np.array_equal(_bits(dres.download(np.float32, rows)), _bits(resid + want))
    # per-block int32 dots through the same dot path
    dots = _buf(rows * (k // 32) * 4)
    _ok(native.camelid_hip_q8_0_block_dots(wq.ptr, rows, k, dxq.ptr, dots.ptr, None))
    assert np.array_equal(dots.download(np.int32, rows * k // 32).reshape(rows, k // 32),
                          orc.q8_0_block_dots(wire, rows, k, xq))


@pytest.mark.parametrize("rows,k,tokens", [(5120, 3072, 130), (3072, 8192, 64), (2048, 5632, 65), (36, 96, 70),
                                           (128, 14336, 3), (1000, 2048, 1), (16384, 3072, 33),
                                           (5120, 3072, 8), (3072, 8192, 5), (36, 2048, 2), (4100, 5632, 7),
                                           # the sweep's prefill batch (512 tokens) and C3's prefill chunk (511)
                                           (2048, 2048, 512), (5632, 2048, 512), (3072, 8192, 511)])
def test_q8_gemm_bit_exact(native, orc, rows, k, tokens):
    """Prefill GEMM on the matrix cores == the per-token GEMV fold of the CPU path."""
    rng = np.random.default_rng(rows + 3 * k + tokens)
    wire = orc.quantize_q8_0_wire(rng.normal(0, 0.02, rows * k).astype(np.float32))
    q, d = _repack(native, wire, rows, k)
    xs = np.empty((tokens, k // 32), np.float32)
    xq = np.empty((tokens, k), np.int8)
    for t in range(tokens):
        xs[t], xq[t] = orc.quantize_q8_0(rng.normal(0, 1 + t % 5, k).astype(np.float32))
    resid = rng.normal(0, 1, (tokens, rows)).astype(np.float32)
    wq, wd, dxq, dxs, dres = _dev(q), _dev(d), _dev(xq), _dev(xs), _dev(resid)
    y = _buf(tokens * rows * 4)
    _ok(native.camelid_hip_q8_0_gemm(wq.ptr, wd.ptr, rows, k, dxq.ptr, dxs.ptr, tokens, y.ptr, None, None))
    got = y.download(np.float32, tokens * rows).reshape(tokens, rows)
    want = np.stack([orc.q8_0_gemv(wire, rows, k, xs[t], xq[t]) for t in range(tokens)])
    assert np.array_equal(_bits(got), _bits(want))
    _ok(native.camelid_hip_q8_0_gemm(wq.ptr, wd.ptr, rows, k, dxq.ptr, dxs.ptr, tokens, dres.ptr, dres.ptr, None))
    assert np.array_equal(_bits(dres.download(np.float32, tokens * rows).reshape(tokens, rows)), _bits(resid + want))


@pytest.mark.parametrize("rows,k,tokens,nf", [(5120, 3072, 130, "2"), (36, 96, 70, "2"), (2048, 5632, 65, "2"),
                                              (32000, 2048, 200, "1"), (4100, 5632, 300, "1")])
def test_q8_gemm_forced_tile_height(native, orc, monkeypatch, rows, k, tokens, nf):
    """The GEMM at the tile height its size would not pick (64 rows for small grids, 32 for a
    large one): the same bits as the CPU fold."""
    monkeypatch.setenv("CAMELID_HIP_GEMM_NF", nf)
    rng = np.random.default_rng(rows + 5 * k + tokens)
    wire = orc.quantize_q8_0_wire(rng.normal(0, 0.02, rows * k).astype(np.float32))
    q, d = _repack(native, wire, rows, k)
    xs = np.empty((tokens, k // 32), np.float32)
    xq = np.empty((tokens, k), np.int8)
    for t in range(tokens):
        xs[t], xq[t] = orc.quantize_q8_0(rng.normal(0, 1 + t % 5, k).astype(np.float32))
    resid = rng.normal(0, 1, (tokens, rows)).astype(np.float32)
    wq, wd, dxq, dxs, dres = _dev(q), _dev(d), _dev(xq), _dev(xs), _dev(resid)
    _ok(native.camelid_hip_q8_0_gemm(wq.ptr, wd.ptr, rows, k, dxq.ptr, dxs.ptr, tokens, dres.ptr, dres.ptr, None))
    want = np.stack([orc.q8_0_gemv(wire, rows, k, xs[t], xq[t]) for t in range(tokens)])
    assert np.array_equal(_bits(dres.download(np.float32, tokens * rows).reshape(tokens, rows)), _bits(resid + want))


@pytest.mark.parametrize("rows,k", [(32000, 2048), (128256, 3072)])
def test_q8_gemm_bit_exact_large(native, orc, rows, k):
    """The sweep's two largest shapes (TinyLlama's and Llama-3.2-3B's lm_head widths) at the
    512-token prefill batch: the whole [512, rows] product on the matrix cores, checked against
    the CPU path's per-token GEMV fold on 384 sampled rows (the first, the last, and rows of
    every 64-row tile position) for every token."""
    from camelid_amd.model import synth_q8_0
    rng = np.random.default_rng(rows + k)
    tokens = 512
    wire = synth_q8_0(f"gemm{rows}x{k}", 2, rows, k, 0.02)
    q, d = _repack(native, wire, rows, k)
    xs = np.empty((tokens, k // 32), np.float32)
    xq = np.empty((tokens, k), np.int8)
    for t in range(tokens):
        xs[t], xq[t] = orc.quantize_q8_0(rng.normal(0, 1 + t % 5, k).astype(np.float32))
    wq, wd, dxq, dxs = _dev(q), _dev(d), _dev(xq), _dev(xs)
    y = _buf(tokens * rows * 4)
    _ok(native.camelid_hip_q8_0_gemm(wq.ptr, wd.ptr, rows, k, dxq.ptr, dxs.ptr, tokens, y.ptr, None, None))
    got = y.download(np.float32, tokens * rows).reshape(tokens, rows)
    sample = np.unique(np.concatenate([[0, rows - 1], np.arange(0, rows, rows // 64)[:64] + np.arange(64) % 64,
                                       rng.choice(rows, 318, replace=False)]))
    rb = k // 32 * 34
    sub = np.ascontiguousarray(wire.reshape(rows, rb)[sample]).ravel()
    want = np.stack([orc.q8_0_gemv(sub, len(sample), k, xs[t], xq[t]) for t in range(tokens)])
    assert np.array_equal(_bits(np.ascontiguousarray(got[:, sample])), _bits(want))


def test_q8_gemm_extreme_quants(native, orc):
    """All -128 quants (largest |int32| block dot), zero-scale rows, through the matrix cores."""
    rows, k, tokens = 64, 1024, 20
    wire = np.zeros((rows, k // 32, 34), np.uint8)
    wire[:, :, :2] = orc.f32_to_f16(np.full((rows, k // 32), 0.5, np.float32)).view(np.uint8).reshape(rows, k // 32, 2)
    wire[:, :, 2:] = np.uint8(0x80)
    wire[::3, :, :2] = 0
    wire = wire.ravel()
    q, d = _repack(native, wire, rows, k)
    xq = np.full((tokens, k), -128, np.int8)
    xq[1::2] = 127
    xs = np.full((tokens, k // 32), 0.25, np.float32)
    wq, wd, dxq, dxs = _dev(q), _dev(d), _dev(xq), _dev(xs)
    y = _buf(rows * tokens * 4)
    _ok(native.camelid_hip_q8_0_gemm(wq.ptr, wd.ptr, rows, k, dxq.ptr, dxs.ptr, tokens, y.ptr, None, None))
    want = np.stack([orc.q8_0_gemv(wire, rows, k, xs[t], xq[t]) for t in range(tokens)])
    assert np.array_equal(_bits(y.download(np.float32, rows * tokens).reshape(tokens, rows)), _bits(want))


@pytest.mark.parametrize("nf", ["1", "2"])
def test_q8_gemm_special_scales(native, orc, monkeypatch, nf):
    """Weight scales across the f16 range through the GEMM's one-FMA fold (the block dots start
    from the bits of 1.5 * 2^23, and fma(f, w, -(1.5 * 2^23) w) gives float(dot) * w): subnormal,
    largest, negative and signed-zero scales, and x scales from f32 subnormals to 1e30.  An
    infinite weight scale (which the one-FMA form cannot give) switches its 16-block staging
    group to the plain conversion and product; the expected +-inf and NaN (dot 0 times inf)
    results come from the CPU fold, compared bit for bit except that any NaN matches any NaN.
    Both tile heights (32 and 64 rows) run."""
    monkeypatch.setenv("CAMELID_HIP_GEMM_NF", nf)
    rows, k, tokens = 128, 2048, 70
    nb = k // 32
    rng = np.random.default_rng(7)
    quants = rng.integers(-128, 128, (rows, nb, 32), dtype=np.int64).astype(np.int8)
    wbits = orc.f32_to_f16(rng.normal(0, 0.02, (rows, nb)).astype(np.float32)).view(np.uint16).copy()
    wbits[5] = rng.integers(1, 0x400, nb)  # f16 subnormals
    wbits[6, ::2], wbits[6, 1::2] = 0x7BFF, 0xFBFF  # +-65504
    wbits[7] |= 0x8000  # negative
    wbits[8, ::2], wbits[8, 1::2] = 0x0000, 0x8000  # +0, -0
    wbits[9, 20] = 0x7C00  # +inf: tile 0, staging group 1
    wbits[70, 40] = 0xFC00  # -inf: tile 1, staging group 2
    wbits[71, 3] = 0x7E00  # NaN (the one-FMA form gives NaN too)
    wire = np.zeros((rows, nb, 34), np.uint8)
    wire[:, :, :2] = wbits.view(np.uint8).reshape(rows, nb, 2)
    wire[:, :, 2:] = quants.view(np.uint8)
    wire = wire.ravel()
    q, d = _repack(native, wire, rows, k)
    xs = np.empty((tokens, nb), np.float32)
    xq = np.empty((tokens, k), np.int8)
    for t in range(tokens):
        xs[t], xq[t] = orc.quantize_q8_0(rng.normal(0, 1 + t % 5, k).astype(np.float32))
    xq[0, 20 * 32:21 * 32] = 0  # dot 0 against the +inf scale: NaN
    xs[1] = np.float32(1e-40)  # f32 subnormal
    xs[2] = np.float32(1e30)
    xs[3, ::3] = 0.0
    wq, wd, dxq, dxs = _dev(q), _dev(d), _dev(xq), _dev(xs)
    y = _buf(rows * tokens * 4)
    _ok(native.camelid_hip_q8_0_gemm(wq.ptr, wd.ptr, rows, k, dxq.ptr, dxs.ptr, tokens, y.ptr, None, None))
    got = y.download(np.float32, rows * tokens).reshape(tokens, rows)
    want = np.stack([orc.q8_0_gemv(wire, rows, k, xs[t], xq[t]) for t in range(tokens)])
    assert np.isnan(want[0, 9]) and np.isinf(want[1:, 9]).any() and np.isinf(want[:, 70]).any()
    diff = (_bits(got) != _bits(want)) & ~(np.isnan(got) & np.isnan(want))
    assert not diff.any(), f"{np.count_nonzero(diff)} mismatches, first at {np.argwhere(diff)[:4].tolist()}"


def test_q8_gemv_extreme_quants(native, orc):
    """All -128 quants on both sides (largest |int32| block dot) and zero scales."""
    rows, k = 64, 1024
    wire = np.zeros((rows, k // 32, 34), np.uint8)
    wire[:, :, :2] = orc.f32_to_f16(np.full((rows, k // 32), 0.5, np.float32)).view(np.uint8).reshape(rows, k // 32, 2)
    wire[:, :, 2:] = np.uint8(0x80)
    wire[::3, :, :2] = 0  # zero scale rows
    wire = wire.ravel()
    q, d = _repack(native, wire, rows, k)
    xq = np.full(k, -128, np.int8)
    xs = np.full(k // 32, 0.25, np.float32)
    wq, wd, dxq, dxs = _dev(q), _dev(d), _dev(xq), _dev(xs)
    y = _buf(rows * 4)
    _ok(native.camelid_hip_q8_0_gemv(wq.ptr, wd.ptr, rows, k, dxq.ptr, dxs.ptr, y.ptr, None, None))
    assert np.array_equal(_bits(y.download(np.float32, rows)), _bits(orc.q8_0_gemv(wire, rows, k, xs, xq)))


def _adversarial_rows(rng, rows, n):
    """Non-negative rows of the kinds that stress the segmented in-order sum: squares of
    normals at many scales, softmax-like exps, constants (round-half-even ties at every
    binade), powers of two, zeros mixed in, subnormal magnitudes, huge leading terms, and
    small integers (exact stretches), plus rows with a negative, infinite or NaN term, all
    zeros, and many negative terms (the plain-step path)."""
    out = np.empty((rows, n), np.float32)
    for r in range(rows):
        kind = r % 13
        scale = np.float32(2.0 ** rng.integers(-30, 30))
        x = rng.normal(0, 1, n).astype(np.float32) * scale
        if kind == 0:
            row = x * x
        elif kind == 1:
            row = np.exp(-np.abs(rng.normal(0, 3, n))).astype(np.float32)
        elif kind == 2:
            row = np.full(n, np.float32(0.75) * scale, np.float32)
        elif kind == 3:
            row = (2.0 ** rng.integers(0, 20, n)).astype(np.float32) * scale
        elif kind == 4:
            row = np.where(rng.random(n) < 0.25, 0, np.abs(x)).astype(np.float32)
        elif kind == 5:
            row = (np.abs(x) * np.float32(2.0 ** -140)).astype(np.float32)
        elif kind == 6:
            row = np.abs(x)
            row[:5] *= np.float32(1e6)
        elif kind == 7:
            row = (rng.integers(0, 64, n) * 2.0 ** rng.integers(0, 8, n)).astype(np.float32)
        elif kind == 8:
            row = x * x
            row[n // 2] = -row[n // 2] if n > 1 else row[0]
        elif kind == 9:
            row = x * x
            if n > 3:
                row[n - 3] = np.inf
        elif kind == 10:
            row = x * x
            row[rng.integers(0, n)] = np.nan
        elif kind == 11:
            row = np.zeros(n, np.float32)
            row[n - 1] = np.float32(1e-45)  # zeros, then the smallest subnormal
        else:
            row = np.where(rng.random(n) < 0.3, -(x * x), x * x).astype(np.float32)
        out[r] = row
    return out


@pytest.mark.parametrize("n", [3072, 2048, 4096, 8192, 16384, 12288, 5000, 768, 257, 256, 129, 7, 1])
def test_inorder_sum_segmented_bit_exact(native, orc, n):
    """The workgroup-parallel exact in-order sum equals the sequential fold bit for bit."""
    rng = np.random.default_rng(n)
    rows = 260 if n <= 4096 else 65
    x = _adversarial_rows(rng, rows, n)
    want = orc.serial_sum_rows(x)
    dx, out = _dev(x), _buf(rows * 4)
    methods = [(0, m) for m in (384, 128, 0, 1)] + [(1, 0)]
    for method, m_seq in methods:
        _ok(native.camelid_hip_inorder_sum_rows(dx.ptr, rows, n, m_seq, method, out.ptr, None))
        got = out.download(np.float32, rows)
        same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (method, m_seq, np.nonzero(~same)[0][:5])


@pytest.mark.parametrize("n", [2048, 3072, 4096, 5120, 8192, 16384, 96])
def test_rmsnorm_quantize_bit_exact(native, orc, n):
    rng = np.random.default_rng(n)
    x = (rng.normal(0, 1, n) * rng.uniform(0.1, 30, n)).astype(np.float32)
    w = rng.normal(1, 0.2, n).astype(np.float32)
    dx, dw = _dev(x), _dev(w)
    xq, xs, y = _buf(n), _buf(n // 32 * 4), _buf(n * 4)
    _ok(native.camelid_hip_rmsnorm_quantize(dx.ptr, dw.ptr, n, 1e-5, xq.ptr, xs.ptr, y.ptr, None))
    want_y = orc.rms_norm(x, w, 1e-5)
    ws, wq = orc.quantize_q8_0(want_y)
    assert np.array_equal(_bits(y.download(np.float32, n)), _bits(want_y))
    assert np.array_equal(_bits(xs.download(np.float32, n // 32)), _bits(ws))
    assert np.array_equal(xq.download(np.int8, n), wq)


def test_quantize_q8_0_bit_exact(native, orc):
    rng = np.random.default_rng(9)
    n = 32 * 5000
    x = rng.normal(0, 1, n).astype(np.float32) * np.repeat(rng.uniform(1e-3, 1e3, n // 32), 32).astype(np.float32)
    x[:32] = 0
    x[32:64] = np.float32(0.5) * np.arange(-16, 16)
    dx, xq, xs = _dev(x), _buf(n), _buf(n // 32 * 4)
    _ok(native.camelid_hip_quantize_q8_0(dx.ptr, n, xq.ptr, xs.ptr, None))
    ws, wq = orc.quantize_q8_0(x)
    assert np.array_equal(_bits(xs.download(np.float32, n // 32)), _bits(ws))
    assert np.array_equal(xq.download(np.int8, n), wq)


def test_silu_mul_quantize_bit_exact(native, orc):
    rng = np.random.default_rng(10)
    n = 8192
    gu = (rng.normal(0, 3, 2 * n)).astype(np.float32)
    gu[:64] = np.linspace(-100, 100, 64)
    dgu, xq, xs, act = _dev(gu), _buf(n), _buf(n // 32 * 4), _buf(n * 4)
    _ok(native.camelid_hip_silu_mul_quantize(dgu.ptr, n, xq.ptr, xs.ptr, act.ptr, None))
    want = orc.silu_mul(gu[:n], gu[n:])
    ws, wq = orc.quantize_q8_0(want)
    assert np.array_equal(_bits(act.download(np.float32, n)), _bits(want))
    assert np.array_equal(_bits(xs.download(np.float32, n // 32)), _bits(ws))
    assert np.array_equal(xq.download(np.int8, n), wq)


@pytest.mark.parametrize("rows,k", [(5120, 3072), (2560, 2048), (6144, 4096), (37, 3072), (8200, 2048)])
def test_rmsnorm_q8_gemv_bit_exact(native, orc, rows, k):
    """The norm computed inside the GEMV == rmsnorm, Q8_0 quantization, then the GEMV."""
    rng = np.random.default_rng(rows + k)
    wire = orc.quantize_q8_0_wire(rng.normal(0, 0.02, rows * k).astype(np.float32))
    q, d = _repack(native, wire, rows, k)
    x = (rng.normal(0, 1, k) * rng.uniform(0.1, 30, k)).astype(np.float32)
    w = rng.normal(1, 0.2, k).astype(np.float32)
    wq, wd, dx, dw, y = _dev(q), _dev(d), _dev(x), _dev(w), _buf(rows * 4)
    _ok(native.camelid_hip_rmsnorm_q8_0_gemv(wq.ptr, wd.ptr, rows, k, dx.ptr, dw.ptr, 1e-5, y.ptr, None))
    xs, xq = orc.quantize_q8_0(orc.rms_norm(x, w, 1e-5))
    assert np.array_equal(_bits(y.download(np.float32, rows)), _bits(orc.q8_0_gemv(wire, rows, k, xs, xq)))


@pytest.mark.parametrize("ffn,k,norm", [(8192, 3072, True), (8192, 3072, False), (5632, 2048, True),
                                        (96, 4096, False), (64, 2048, False), (96, 3072, True),
                                        (14336, 4096, True), (12288, 4096, True)])
def test_gate_up_silu_bit_exact(native, orc, ffn, k, norm):
    """Fused gate/up GEMV + SwiGLU + Q8_0 of the activation (rows interleaved by 32)."""
    rng = np.random.default_rng(ffn + k + norm)
    gate = rng.normal(0, 0.02, (ffn, k)).astype(np.float32)
    up = rng.normal(0, 0.02, (ffn, k)).astype(np.float32)
    inter = np.concatenate([gate.reshape(ffn // 32, 32, k), up.reshape(ffn // 32, 32, k)], axis=1)
    wire = orc.quantize_q8_0_wire(inter.reshape(-1))
    q, d = _repack(native, wire, 2 * ffn, k)
    x = (rng.normal(0, 1, k) * rng.uniform(0.1, 30, k)).astype(np.float32)
    w = rng.normal(1, 0.2, k).astype(np.float32)
    xs, xq = orc.quantize_q8_0(orc.rms_norm(x, w, 1e-5))
    wq, wd, aq, as_ = _dev(q), _dev(d), _buf(ffn), _buf(ffn // 32 * 4)
    if norm:
        dx, dw = _dev(x), _dev(w)
        _ok(native.camelid_hip_gate_up_silu(wq.ptr, wd.ptr, ffn, k, None, None, dx.ptr, dw.ptr, 1e-5, aq.ptr,
                                            as_.ptr, None))
    else:
        dxq, dxs = _dev(xq), _dev(xs)
        _ok(native.camelid_hip_gate_up_silu(wq.ptr, wd.ptr, ffn, k, dxq.ptr, dxs.ptr, None, None, 0.0, aq.ptr,
                                            as_.ptr, None))
    rows_out = orc.q8_0_gemv(wire, 2 * ffn, k, xs, xq).reshape(ffn // 32, 2, 32)
    act = orc.silu_mul(rows_out[:, 0].reshape(-1), rows_out[:, 1].reshape(-1))
    ws, wq8 = orc.quantize_q8_0(act)
    assert np.array_equal(_bits(as_.download(np.float32, ffn // 32)), _bits(ws))
    assert np.array_equal(aq.download(np.int8, ffn), wq8)


def _kv_device(k, v):
    """[L][n_kv][kvs][hd] K and V (f16 bits) -> the device layout: K granules of 8 dims per
    position ([hd/8][kvs][8]), V granules of 8 positions per dim ([kvs/8][hd][8])."""
    L, nkv, kvs, hd = k.shape
    kd = k.reshape(L, nkv, kvs, hd // 8, 8).transpose(0, 1, 3, 2, 4)
    vd = v.reshape(L, nkv, kvs // 8, 8, hd).transpose(0, 1, 2, 4, 3)
    return np.ascontiguousarray(kd), np.ascontiguousarray(vd)


def _kv_host(kd, vd, L, nkv, kvs, hd):
    """Inverse of _kv_device, from the flat device arrays."""
    k = kd.reshape(L, nkv, hd // 8, kvs, 8).transpose(0, 1, 3, 2, 4).reshape(L, nkv, kvs, hd)
    v = vd.reshape(L, nkv, kvs // 8, hd, 8).transpose(0, 1, 2, 4, 3).reshape(L, nkv, kvs, hd)
    return k, v


def test_kv_layout_helpers_roundtrip():
    rng = np.random.default_rng(0)
    k = rng.integers(0, 65535, (2, 3, 16, 64)).astype(np.uint16)
    v = rng.integers(0, 65535, (2, 3, 16, 64)).astype(np.uint16)
    kd, vd = _kv_device(k, v)
    # spot-check the index formulas: K (p, d) at ((d/8)*kvs + p)*8 + d%8, V at ((p/8)*hd + d)*8 + p%8
    kf, vf = kd.reshape(2, 3, -1), vd.reshape(2, 3, -1)
    for p_, d_ in [(0, 0), (5, 13), (15, 63), (8, 7), (9, 1)]:
        assert kf[1, 2, ((d_ // 8) * 16 + p_) * 8 + d_ % 8] == k[1, 2, p_, d_]
        assert vf[1, 2, ((p_ // 8) * 64 + d_) * 8 + p_ % 8] == v[1, 2, p_, d_]
    k2, v2 = _kv_host(kd.ravel(), vd.ravel(), 2, 3, 16, 64)
    assert np.array_equal(k2, k) and np.array_equal(v2, v)


@pytest.mark.parametrize("nh,nkv,hd,split,qk", [(24, 8, 128, False, False), (32, 4, 64, False, False),
                                                (32, 8, 128, True, True)])
def test_rope_kv_bit_exact(native, orc, nh, nkv, hd, split, qk):
    rng = np.random.default_rng(nh + hd)
    L, max_pos, layer, pos = 2, 40, 1, 33  # max_pos (the position stride) is a multiple of 8
    qkv = rng.normal(0, 2, (nh + 2 * nkv) * hd).astype(np.float32)
    c, s = orc.rope_tables(hd, 500000.0, 2, 32.0, 8192.0, 1.0, 4.0, None, pos, 1)
    qn = rng.normal(1, 0.3, hd).astype(np.float32) if qk else None
    kn = rng.normal(1, 0.3, hd).astype(np.float32) if qk else None
    kc = _buf(L * nkv * max_pos * hd * 2)
    vc = _buf(L * nkv * max_pos * hd * 2)
    qrot = _buf(nh * hd * 4)
    dq, dc, ds, dpos = _dev(qkv), _dev(c[0]), _dev(s[0]), _dev(np.array([pos], np.uint32))
    dqn = _dev(qn) if qk else None
    dkn = _dev(kn) if qk else None
    _ok(native.camelid_hip_rope_kv(dq.ptr, nh, nkv, hd, hd, int(split), dc.ptr, ds.ptr,
                                   dqn.ptr if qk else None, dkn.ptr if qk else None, 1e-5, qrot.ptr, kc.ptr, vc.ptr,
                                   layer, max_pos, dpos.ptr, None))
    q = qkv[:nh * hd]
    k = qkv[nh * hd:(nh + nkv) * hd]
    v = qkv[(nh + nkv) * hd:]
    if qk:
        q = orc.rms_norm(q.reshape(nh, hd), qn, 1e-5).ravel()
        k = orc.rms_norm(k.reshape(nkv, hd), kn, 1e-5).ravel()
    want_q = orc.apply_rope(q, nh, hd, hd, c[0], s[0], split)
    want_k = orc.apply_rope(k, nkv, hd, hd, c[0], s[0], split)
    assert np.array_equal(_bits(qrot.download(np.float32, nh * hd)), _bits(want_q))
    kk, vv = _kv_host(kc.download(np.uint16, L * nkv * max_pos * hd), vc.download(np.uint16, L * nkv * max_pos * hd),
                      L, nkv, max_pos, hd)
    assert np.array_equal(kk[layer, :, pos], orc.f32_to_f16(want_k).reshape(nkv, hd))
    assert np.array_equal(vv[layer, :, pos], orc.f32_to_f16(v).reshape(nkv, hd))


@pytest.mark.parametrize("nh,nkv,hd,P", [(24, 8, 128, 1), (24, 8, 128, 2), (24, 8, 128, 9), (24, 8, 128, 511),
                                         (24, 8, 128, 767), (32, 4, 64, 129), (8, 8, 64, 300), (32, 8, 128, 1280),
                                         (32, 8, 128, 2100), (8, 4, 256, 700), (8, 4, 256, 40),
                                         (32, 8, 128, 5000), (32, 8, 128, 8448), (8, 4, 256, 3000),
                                         (32, 8, 64, 12000), (32, 8, 128, 4000), (32, 8, 128, 6200),
                                         (8, 4, 128, 13000)])
def test_attention_decode_bit_exact(native, orc, nh, nkv, hd, P):
    rng = np.random.default_rng(P + nh)
    L, layer, max_pos = 2, 1, (max(P, 2) + 3 + 7) // 8 * 8  # position stride: multiple of 8
    kf = rng.normal(0, 1.5, (L, nkv, max_pos, hd)).astype(np.float32)
    vf = rng.normal(0, 1, (L, nkv, max_pos, hd)).astype(np.float32)
    kb, vb = orc.f32_to_f16(kf), orc.f32_to_f16(vf)
    q = rng.normal(0, 1, nh * hd).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    kd, vd = _kv_device(kb, vb)
    dq, dk, dv = _dev(q), _dev(kd), _dev(vd)
    dpos = _dev(np.array([P - 1], np.uint32))
    out, xq, xs = _buf(nh * hd * 4), _buf(nh * hd), _buf(nh * hd // 32 * 4)
    want = orc.attention(q, orc.f16_to_f32(kb[layer]).ravel(), orc.f16_to_f32(vb[layer]).ravel(), nh, nkv, hd,
                         max_pos, P)
    ws, wq = orc.quantize_q8_0(want)
    # one workgroup per head, and the long-context split over workgroups
    for entry in (native.camelid_hip_attention_decode, native.camelid_hip_attention_decode_split):
        _ok(entry(dq.ptr, dk.ptr, dv.ptr, layer, nh, nkv, hd, max_pos, dpos.ptr, scale, out.ptr, xq.ptr, xs.ptr, None))
        assert np.array_equal(_bits(out.download(np.float32, nh * hd)), _bits(want))
        assert np.array_equal(_bits(xs.download(np.float32, nh * hd // 32)), _bits(ws))
        assert np.array_equal(xq.download(np.int8, nh * hd), wq)


@pytest.mark.parametrize("tiled", [True, False])
@pytest.mark.parametrize("nh,nkv,hd,pos0,T", [(24, 8, 128, 0, 70), (24, 8, 128, 500, 11), (32, 4, 64, 3, 130),
                                             (8, 4, 256, 40, 9), (4, 4, 64, 0, 1), (32, 8, 128, 8000, 20),
                                             (24, 8, 128, 700, 64), (4, 4, 64, 0, 200), (32, 8, 128, 61, 33)])
def test_attention_prefill_bit_exact(native, orc, monkeypatch, nh, nkv, hd, pos0, T, tiled):
    """Causal attention of a prefill chunk == the decode attention of each of its tokens, for
    the tiled kernel (a tile's rows sharing K/V blocks, rows ending inside a block, rows of one
    position) and the one-workgroup-per-(head, token) kernel (CAMELID_HIP_ATT_TILE=0); head_dim
    256 runs the latter either way."""
    monkeypatch.setenv("CAMELID_HIP_ATT_TILE", "1" if tiled else "0")
    rng = np.random.default_rng(pos0 * 31 + T + hd)
    L, layer = 2, 1
    max_pos = (pos0 + T + 5 + 7) // 8 * 8
    kf = rng.normal(0, 1.5, (L, nkv, max_pos, hd)).astype(np.float32)
    vf = rng.normal(0, 1, (L, nkv, max_pos, hd)).astype(np.float32)
    kb, vb = orc.f32_to_f16(kf), orc.f32_to_f16(vf)
    q = rng.normal(0, 1, (T, nh * hd)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    kd, vd = _kv_device(kb, vb)
    dq, dk, dv = _dev(q), _dev(kd), _dev(vd)
    out, xq, xs = _buf(T * nh * hd * 4), _buf(T * nh * hd), _buf(T * nh * hd // 32 * 4)
    _ok(native.camelid_hip_attention_prefill(dq.ptr, dk.ptr, dv.ptr, layer, nh, nkv, hd, max_pos, pos0, T, scale,
                                             out.ptr, xq.ptr, xs.ptr, None))
    got = out.download(np.float32, T * nh * hd).reshape(T, nh * hd)
    gxq = xq.download(np.int8, T * nh * hd).reshape(T, nh * hd)
    gxs = xs.download(np.float32, T * nh * hd // 32).reshape(T, nh * hd // 32)
    kl, vl = orc.f16_to_f32(kb[layer]).ravel(), orc.f16_to_f32(vb[layer]).ravel()
    for t in range(T):
        want = orc.attention(q[t], kl, vl, nh, nkv, hd, max_pos, pos0 + t + 1)
        assert np.array_equal(_bits(got[t]), _bits(want)), f"token {t}"
        ws, wq = orc.quantize_q8_0(want)
        assert np.array_equal(_bits(gxs[t]), _bits(ws)) and np.array_equal(gxq[t], wq)


def test_quantize_q8_k_bit_exact(native, orc):
    """Q8_K activation quantizer == quantize_q8_k_blocks, incl. zero blocks, |max| ties (first
    wins), one-hot and huge/tiny blocks; per-32 sums of the quants."""
    rng = np.random.default_rng(41)
    nb = 64
    x = rng.normal(0, 1, nb * 256).astype(np.float32)
    b = x.reshape(nb, 256)
    b[1] = 0.0
    b[2] = rng.uniform(-1, 1, 256); b[2, 7], b[2, 200] = -3.0, 3.0
    b[3] = rng.uniform(-1, 1, 256); b[3, 100], b[3, 20] = 3.0, -3.0
    b[4] = 0.0; b[4, 255] = 1e-30
    b[5] *= 1e30
    b[6] = np.round(rng.normal(0, 40, 256)) / 127.0      # many exact .5 products: round-half-even
    b[7] = -1.0
    dx = _dev(x)
    yd, yq, ybs = _buf(nb * 4), _buf(nb * 256), _buf(nb * 8 * 4)
    _ok(native.camelid_hip_quantize_q8_k(dx.ptr, nb * 256, yd.ptr, yq.ptr, ybs.ptr, None))
    wd, wq = orc.quantize_q8_k(x)
    assert np.array_equal(_bits(yd.download(np.float32, nb)), _bits(wd))
    gq = yq.download(np.int8, nb * 256)
    assert np.array_equal(gq, wq)
    assert np.array_equal(ybs.download(np.int32, nb * 8), wq.astype(np.int64).reshape(-1, 32).sum(1))


@pytest.mark.parametrize("n", [4096, 3072, 256, 16384])
def test_rmsnorm_and_silu_q8_k_bit_exact(native, orc, n):
    """The Q8_K activation written by the RMSNorm and SwiGLU kernels == the CPU norm / SwiGLU
    followed by quantize_q8_k_blocks."""
    rng = np.random.default_rng(n + 7)
    x = rng.normal(0, 1, n).astype(np.float32)
    x[:256] *= 1e-3
    w = rng.normal(1, 0.1, n).astype(np.float32)
    yd, yq, ybs = _buf(n // 256 * 4), _buf(n), _buf(n // 32 * 4)
    dx, dw = _dev(x), _dev(w)  # the buffers must outlive the launch
    _ok(native.camelid_hip_rmsnorm_q8_k(dx.ptr, dw.ptr, n, 1e-5, yd.ptr, yq.ptr, ybs.ptr, None))
    wd, wq = orc.quantize_q8_k(orc.rms_norm(x, w, 1e-5))
    assert np.array_equal(_bits(yd.download(np.float32, n // 256)), _bits(wd))
    assert np.array_equal(yq.download(np.int8, n), wq)
    assert np.array_equal(ybs.download(np.int32, n // 32), wq.astype(np.int64).reshape(-1, 32).sum(1))
    gu = rng.normal(0, 2, 2 * n).astype(np.float32)
    dgu = _dev(gu)
    _ok(native.camelid_hip_silu_mul_q8_k(dgu.ptr, n, yd.ptr, yq.ptr, ybs.ptr, None))
    wd, wq = orc.quantize_q8_k(orc.silu_mul(gu[:n], gu[n:]))
    assert np.array_equal(_bits(yd.download(np.float32, n // 256)), _bits(wd))
    assert np.array_equal(yq.download(np.int8, n), wq)
    assert np.array_equal(ybs.download(np.int32, n // 32), wq.astype(np.int64).reshape(-1, 32).sum(1))


def _kquant_wire(orc, rng, quant, rows, k):
    """Random superblocks with finite f16 scales (every other byte uniformly random)."""
    nsb, bb = k // 256, (144 if quant == 1 else 210)
    wire = rng.integers(0, 256, (rows, nsb, bb), dtype=np.uint8)
    if quant == 1:
        wire[:, :, 0:4] = orc.f32_to_f16(rng.uniform(-2e-3, 2e-3, (rows, nsb, 2)).astype(np.float32)).view(
            np.uint8).reshape(rows, nsb, 4)
    else:
        wire[:, :, 208:210] = orc.f32_to_f16(rng.uniform(-2e-3, 2e-3, (rows, nsb)).astype(np.float32)).view(
            np.uint8).reshape(rows, nsb, 2)
    return wire.ravel()


def _kquant_planes(native, quant, wire, rows, k):
    from camelid_amd._native import ptr
    nsb = k // 256
    a = np.empty(rows * k // 2, np.uint8)
    b = np.empty(rows * nsb * (16 if quant == 1 else 64), np.uint8)
    sc = np.empty(max(rows * nsb * 16, 1), np.int8)
    d = np.empty(max(rows * nsb, 1), np.uint16)
    _ok(native.camelid_kquant_repack(quant, ptr(wire, C.c_uint8), rows, k, ptr(a, C.c_uint8), ptr(b, C.c_uint8),
                                     ptr(sc, C.c_int8), ptr(d, C.c_uint16)))
    return _dev(a), _dev(b), _dev(sc), _dev(d)


@pytest.mark.parametrize("quant,rows,k", [(1, 4096, 4096), (1, 12288, 4096), (1, 4096, 12288), (1, 36, 256),
                                          (1, 16384, 2048), (2, 1024, 4096), (2, 20000, 4096), (2, 37, 512),
                                          (2, 4096, 12288)])
def test_kquant_gemv_bit_exact(native, orc, quant, rows, k):
    """Q4_K (q4_k_dot_arm order) / Q6_K (8-lane q6_k_wire_row_dot order) GEMV == the CPU dots."""
    rng = np.random.default_rng(rows + k + quant)
    wire = _kquant_wire(orc, rng, quant, rows, k)
    ydh, yqh = orc.quantize_q8_k(rng.normal(0, 1, k).astype(np.float32))
    bsh = yqh.astype(np.int32).reshape(-1, 32).sum(1).astype(np.int32)
    a, b, sc, d = _kquant_planes(native, quant, wire, rows, k)
    yd, yq, ybs = _dev(ydh), _dev(yqh), _dev(bsh)
    resid = rng.normal(0, 1, rows).astype(np.float32)
    dres, y = _dev(resid), _buf(rows * 4)
    _ok(native.camelid_hip_kquant_gemv(quant, a.ptr, b.ptr, sc.ptr, d.ptr, rows, k, yd.ptr, yq.ptr, ybs.ptr, y.ptr,
                                       None, None))
    want = orc.kquant_gemv(quant, wire, rows, k, ydh, yqh)
    assert np.array_equal(_bits(y.download(np.float32, rows)), _bits(want))
    _ok(native.camelid_hip_kquant_gemv(quant, a.ptr, b.ptr, sc.ptr, d.ptr, rows, k, yd.ptr, yq.ptr, ybs.ptr,
                                       dres.ptr, dres.ptr, None))
    assert np.array_equal(_bits(dres.download(np.float32, rows)), _bits(resid + want))


@pytest.mark.parametrize("quant,rows,k,T,ldy", [(1, 64, 256, 1, 64), (1, 100, 512, 5, 100), (1, 1024, 4096, 8, 1024),
                                                 (1, 4096, 4096, 70, 4100), (1, 300, 12288, 3, 300),
                                                 (1, 2048, 4096, 130, 2048), (1, 36, 16384, 65, 40),
                                                 (2, 1024, 4096, 8, 1024), (2, 37, 512, 13, 50),
                                                 (2, 300, 12288, 5, 300), (2, 2048, 4096, 20, 2048),
                                                 (2, 1024, 4096, 130, 1024), (2, 100, 12288, 33, 104)])
def test_kquant_gemm_bit_exact(native, orc, quant, rows, k, T, ldy):
    """Multi-token K-quant projection (Q4_K on the matrix cores; Q6_K on the matrix cores above 8
    tokens, by the multi-token GEMV up to 8): every
    (token, row) equals the single-token GEMV on that token bit for bit (and the CPU dot on
    the first and last token), with a strided, residual-carrying output; ragged row and token
    tiles, K up to 16384."""
    rng = np.random.default_rng(rows * 7 + k + T + quant)
    wire = _kquant_wire(orc, rng, quant, rows, k)
    a, b, sc, d = _kquant_planes(native, quant, wire, rows, k)
    x = rng.normal(0, 1, (T, k)).astype(np.float32)
    x[T // 2, : k // 3] = 0.0  # a token with all-zero Q8_K blocks
    yds, yqs = zip(*(orc.quantize_q8_k(x[t]) for t in range(T)))
    ydh, yqh = np.stack(yds).astype(np.float32), np.stack(yqs).astype(np.int8)
    yd, yq = _dev(ydh), _dev(yqh)
    resid = rng.normal(0, 1, (T, ldy)).astype(np.float32)
    dres, y = _dev(resid), _buf(T * ldy * 4)
    _ok(native.camelid_hip_kquant_gemm(quant, a.ptr, b.ptr, sc.ptr, d.ptr, rows, k, T, yd.ptr, yq.ptr, y.ptr, ldy,
                                       None, None))
    got = y.download(np.float32, T * ldy).reshape(T, ldy)[:, :rows]
    _ok(native.camelid_hip_kquant_gemm(quant, a.ptr, b.ptr, sc.ptr, d.ptr, rows, k, T, yd.ptr, yq.ptr, dres.ptr, ldy,
                                       dres.ptr, None))
    got_r = dres.download(np.float32, T * ldy).reshape(T, ldy)
    one, ybs = _buf(rows * 4), _buf(k // 32 * 4)
    for t in range(T):
        tyd, tyq = _dev(ydh[t]), _dev(yqh[t])
        dbs = _dev(yqh[t].astype(np.int32).reshape(-1, 32).sum(1).astype(np.int32))
        _ok(native.camelid_hip_kquant_gemv(quant, a.ptr, b.ptr, sc.ptr, d.ptr, rows, k, tyd.ptr, tyq.ptr, dbs.ptr,
                                           one.ptr, None, None))
        want = one.download(np.float32, rows)
        assert np.array_equal(_bits(got[t]), _bits(want)), f"token {t}"
        assert np.array_equal(_bits(got_r[t, :rows]), _bits(resid[t, :rows] + want)), f"token {t} (resid)"
        assert np.array_equal(_bits(got_r[t, rows:]), _bits(resid[t, rows:])), "past the rows"
        if t in (0, T - 1):
            assert np.array_equal(_bits(want), _bits(orc.kquant_gemv(quant, wire, rows, k, ydh[t], yqh[t])))


@pytest.mark.parametrize("case", ["min", "max", "mixed"])
def test_q6k_gemm_extreme_products(native, orc, case):
    """Q6_K chunk GEMM at the ends of its integer range: scaled weights sc * w of +4096 (sc =
    -128, w = -32) and 127 * 31 against Q8_K quants of -127 and +127, so a class's integer dot
    reaches 32 * 4096 * 127 (just under 2^24); every (token, row) equals the single-token GEMV
    and the CPU dot bit for bit."""
    rows, k, T = 64, 512, 40
    rng = np.random.default_rng(7)
    wire = _kquant_wire(orc, rng, 2, rows, k).reshape(rows, k // 256, 210)
    if case == "min":  # ql = qh = 0: w = -32 everywhere; sc = -128
        wire[:, :, 0:192] = 0
        wire[:, :, 192:208] = np.uint8(0x80)
    elif case == "max":  # ql = qh = all ones: w = 31; sc = 127
        wire[:, :, 0:192] = 0xFF
        wire[:, :, 192:208] = 127
    else:  # per superblock one of the two extremes, scales at +-127 / -128
        wire[::2, :, 0:192] = 0
        wire[1::2, :, 0:192] = 0xFF
        wire[:, :, 192:208] = rng.choice(np.array([0x80, 0x7F, 0x81], np.uint8), (rows, k // 256, 16))
    wire = wire.ravel()
    a, b, sc, d = _kquant_planes(native, 2, wire, rows, k)
    x = np.ones((T, k), np.float32)  # quants of -127 (a block's max maps to -127 whatever its sign)
    x[1::3] = -1.0
    x[1::3, ::256] = 1.0  # each block's first element is its max: the -1 entries give +127
    x[2::5, ::7] = 0.5
    yds, yqs = zip(*(orc.quantize_q8_k(x[t]) for t in range(T)))
    ydh, yqh = np.stack(yds).astype(np.float32), np.stack(yqs).astype(np.int8)
    assert (yqh == -127).any() and (yqh == 127).any()
    yd, yq, y = _dev(ydh), _dev(yqh), _buf(T * rows * 4)
    _ok(native.camelid_hip_kquant_gemm(2, a.ptr, b.ptr, sc.ptr, d.ptr, rows, k, T, yd.ptr, yq.ptr, y.ptr, rows,
                                       None, None))
    got = y.download(np.float32, T * rows).reshape(T, rows)
    one, ybs = _buf(rows * 4), _buf(k // 32 * 4)
    for t in range(T):
        tyd, tyq = _dev(ydh[t]), _dev(yqh[t])
        dbs = _dev(yqh[t].astype(np.int32).reshape(-1, 32).sum(1).astype(np.int32))
        _ok(native.camelid_hip_kquant_gemv(2, a.ptr, b.ptr, sc.ptr, d.ptr, rows, k, tyd.ptr, tyq.ptr, dbs.ptr,
                                           one.ptr, None, None))
        want = one.download(np.float32, rows)
        assert np.array_equal(_bits(got[t]), _bits(want)), f"token {t}"
        if t in (0, 1, T - 1):
            assert np.array_equal(_bits(want), _bits(orc.kquant_gemv(2, wire, rows, k, ydh[t], yqh[t])))


@pytest.mark.parametrize("n", [1, 1000, 32000, 128256, 151936])
def test_argmax_matches_first_max(native, orc, n):
    rng = np.random.default_rng(n)
    x = rng.integers(-50, 50, n).astype(np.float32)  # heavy ties: first index must win
    dx, out = _dev(x), _buf(4)
    _ok(native.camelid_hip_argmax(dx.ptr, n, out.ptr, None))
    assert int(out.download(np.uint32, 1)[0]) == orc.argmax(x) == int(np.argmax(x))
    x = np.full(n, -np.inf, np.float32)
    dx = _dev(x)
    _ok(native.camelid_hip_argmax(dx.ptr, n, out.ptr, None))
    assert int(out.download(np.uint32, 1)[0]) == 0
