"""Pins of the CPU oracle (oracle/camelid_oracle.cpp) -- CPU only.

Each oracle function is checked against something that does not restate it: the
reference's own golden fixtures (tests/fixtures/dequant/*.json, gguf==0.19.0), ported
known-answer tests from the reference's test suite, exhaustive/brute-force checks, and
closed forms or float64 bounds chosen so a dropped term, wrong sign or transposed
operand fails.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

GOLD = Path(__file__).resolve().parent / "golden" / "reference_dequant"


def _fixture(name):
    d = json.loads((GOLD / name).read_text())
    raw = np.frombuffer(bytes.fromhex(d["quant_hex"]), np.uint8)
    ref = np.array([int(x, 16) for x in d["ref_f32_bits"]], np.uint32)
    return d, raw, ref


# ------------------------------------------------------------------ f16 conversions
def test_f16_fixture_matches_reference(orc):
    _, raw, ref = _fixture("F16.json")
    got = orc.f16_to_f32(raw.view(np.uint16)).view(np.uint32)
    assert np.array_equal(got, ref)


def test_f16_to_f32_exhaustive_matches_ieee(orc):
    # kv_f16.rs:215-268 asserts equality with F16C over all halves; numpy's widening is exact.
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(allh)
    want = allh.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))


def test_f32_to_f16_matches_ieee_rne(orc):
    rng = np.random.default_rng(0)
    # every half value, its neighbours and the midpoints between halves, plus random bits
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    halves = halves[np.isfinite(halves)]
    bits = halves.view(np.uint32)
    cand = np.concatenate([bits, bits + 1, bits - 1, bits + 0x1000, bits + 0xfff, bits + 0x1001,
                           rng.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32)])
    x = cand.view(np.float32)
    x = x[~np.isnan(x)]
    got = orc.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # NaN canonicalises to 0x7e00 with the sign kept (inference.rs:20775)
    assert orc.f32_to_f16(np.array([np.nan], np.float32))[0] & 0x7fff == 0x7e00


# ------------------------------------------------------------------ Q8_0
def test_q8_0_dequant_fixture_matches_reference(orc):
    _, raw, ref = _fixture("Q8_0.json")
    got = orc.dequant_q8_0_wire(raw).view(np.uint32)
    assert np.array_equal(got, ref)


def test_quantize_uses_unrounded_scale_for_quants(orc):
    # Port of inference/tests.rs:2570 q8_0_input_quantization_uses_unrounded_scale_for_quants.
    unrounded = np.float32(1.0) / np.float32(127.0)
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    x[1] = np.float32(2.49995) * unrounded
    s, q = orc.quantize_q8_0(x)
    assert s[0] == orc.f16_to_f32(orc.f32_to_f16(np.array([unrounded], np.float32)))[0]
    assert q[0] == 127
    assert q[1] == 2
    assert int(np.round(x[1] / s[0])) == 3


def test_quantize_properties(orc):
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, 32 * 4096).astype(np.float32)
    x[:32] = 0.0                                   # all-zero block -> scale 0, quants 0
    x[32:64] = np.float32(0.5) * np.arange(-16, 16, dtype=np.float32)  # exact halves -> round away from zero
    s, q = orc.quantize_q8_0(x)
    xb = x.reshape(-1, 32).astype(np.float64)
    amax = np.abs(xb).max(1)
    unrounded = (amax.astype(np.float32) / np.float32(127)).astype(np.float32)
    assert np.array_equal(s, orc.f16_to_f32(orc.f32_to_f16(unrounded)))
    assert s[0] == 0 and np.all(q[:32] == 0)
    # the element with |x| == amax quantizes to +-127 (or -128 never: amax maps to 127)
    qb = q.reshape(-1, 32).astype(np.int32)
    assert np.all(np.abs(qb).max(1)[1:] == 127)
    # |x*inv - q| <= 0.5 everywhere (rounding), q within [-128, 127]
    inv = np.where(unrounded == 0, 0, 1.0 / unrounded.astype(np.float64))
    err = np.abs(xb * inv[:, None] - qb)
    assert err.max() <= 0.5 + 1e-4
    # block 1: amax = 8, inv = 127/8 -> x*inv = k*0.5*15.875; ties would round away from zero
    assert q[32] == -127 and q[63] == int(np.round(7.5 * 15.875 + 1e-9))


def test_block_int_dot_brute_force(orc):
    rng = np.random.default_rng(2)
    w = rng.integers(-128, 128, (500, 32)).astype(np.int8)
    x = rng.integers(-128, 128, (500, 32)).astype(np.int8)
    w[0] = -128
    x[0] = -128  # extreme: 32 * 16384
    for i in range(500):
        assert orc.lib().oracle_q8_block_dot(orc.P(w[i], orc.C.c_int8), orc.P(x[i], orc.C.c_int8)) == \
            int(np.dot(w[i].astype(np.int64), x[i].astype(np.int64)))


def _rand_q8_matrix(orc, rng, rows, k, scale_pow2=False):
    if scale_pow2:
        # power-of-two scales and small ints: every product and partial sum is exact in f32
        q = rng.integers(-3, 4, (rows, k)).astype(np.int8)
        wire = np.zeros((rows, k // 32, 34), np.uint8)
        e = rng.integers(-4, 2, (rows, k // 32))
        sc = (2.0 ** e).astype(np.float32)
        wire[:, :, :2] = orc.f32_to_f16(sc).view(np.uint8).reshape(rows, k // 32, 2)
        wire[:, :, 2:] = q.reshape(rows, k // 32, 32).view(np.uint8)
        return wire.ravel(), q.astype(np.float64), np.repeat(sc.astype(np.float64), 32, axis=1)
    w = rng.normal(0, 0.02, rows * k).astype(np.float32)
    wire = orc.quantize_q8_0_wire(w)
    deq = orc.dequant_q8_0_wire(wire).reshape(rows, k).astype(np.float64)
    return wire, deq, None


def test_gemv_exact_case_equals_integer_arithmetic(orc):
    rng = np.random.default_rng(3)
    rows, k = 64, 512
    wire, q, sc = _rand_q8_matrix(orc, rng, rows, k, scale_pow2=True)
    xq = rng.integers(-3, 4, k).astype(np.int8)
    xs = (2.0 ** rng.integers(-3, 1, k // 32)).astype(np.float32)
    got = orc.q8_0_gemv(wire, rows, k, xs, xq)
    want = (q * sc * (xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32))[None, :]).sum(1)
    assert np.array_equal(got.astype(np.float64), want)


def test_gemv_float64_bound_and_block_dots(orc):
    rng = np.random.default_rng(4)
    rows, k = 300, 1024
    wire, deq, _ = _rand_q8_matrix(orc, rng, rows, k)
    x = rng.normal(0, 1, k).astype(np.float32)
    xs, xq = orc.quantize_q8_0(x)
    got = orc.q8_0_gemv(wire, rows, k, xs, xq).astype(np.float64)
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    terms = deq * xd[None, :]
    exact = terms.sum(1)
    bound = (k // 32 + 2) * 2.0 ** -23 * np.abs(terms).sum(1) + 1e-30
    assert np.all(np.abs(got - exact) <= bound)
    # per-block int dots against brute force
    dots = orc.q8_0_block_dots(wire, rows, k, xq)
    qw = np.frombuffer(wire.tobytes(), np.uint8).reshape(rows, k // 32, 34)[:, :, 2:].view(np.int8).astype(np.int64)
    want = (qw * xq.reshape(k // 32, 32).astype(np.int64)[None]).sum(2)
    assert np.array_equal(dots, want)
    # batched form is the same fold per token
    X = rng.normal(0, 1, (3, k)).astype(np.float32)
    q3 = [orc.quantize_q8_0(X[t]) for t in range(3)]
    G = orc.q8_0_gemm(wire, rows, k, np.stack([a for a, _ in q3]), np.stack([b for _, b in q3]))
    for t in range(3):
        assert np.array_equal(G[t], orc.q8_0_gemv(wire, rows, k, q3[t][0], q3[t][1]))


# ------------------------------------------------------------------ RMSNorm
def test_rms_norm_closed_form_and_bound(orc):
    n = 3072
    x = np.full(n, 0.75, np.float32)       # ms = 0.5625 exactly; all partial sums exact
    w = np.ones(n, np.float32)
    y = orc.rms_norm(x, w, 1e-5)
    s = np.float32(1.0) / np.sqrt(np.float32(0.5625) + np.float32(1e-5))
    assert np.all(y == np.float32(0.75) * s)
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, n).astype(np.float32)
    w = rng.normal(1, 0.1, n).astype(np.float32)
    y = orc.rms_norm(x, w, 1e-5).astype(np.float64)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5) * w
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-30)) < 5e-5
    # scaling the input by 2 leaves the output (nearly) unchanged: catches a missing sqrt/mean
    y2 = orc.rms_norm(2 * x, w, 0.0).astype(np.float64)
    y1 = orc.rms_norm(x, w, 0.0).astype(np.float64)
    assert np.max(np.abs(y2 - y1)) < 1e-5


# ------------------------------------------------------------------ RoPE
def test_rope_pos0_identity_and_norm(orc):
    c, s = orc.rope_tables(128, 500000.0, 2, 32.0, 8192.0, 1.0, 4.0, None, 0, 3)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, 4 * 128).astype(np.float32)
    assert np.array_equal(orc.apply_rope(x, 4, 128, 128, c[0], s[0]), x)
    for split in (False, True):
        y = orc.apply_rope(x, 4, 128, 128, c[2], s[2], split).astype(np.float64)
        if split:
            a = x.reshape(4, 2, 64)
            b = y.reshape(4, 2, 64)
            na = (a.astype(np.float64) ** 2).sum(1)
            nb_ = (b ** 2).sum(1)
        else:
            na = (x.reshape(4, 64, 2).astype(np.float64) ** 2).sum(2)
            nb_ = (y.reshape(4, 64, 2) ** 2).sum(2)
        assert np.allclose(na, nb_, rtol=1e-5)


def test_rope_configured_base_kat(orc):
    # Port of inference/tests.rs:8397 apply_rope_uses_configured_frequency_base.
    c, s = orc.rope_tables(4, 500000.0, 0, pos0=1, n_pos=1)
    y = orc.apply_rope(np.array([0, 0, 1, 0], np.float32), 1, 4, 4, c[0], s[0])
    th = np.float32(500000.0) ** np.float32(-0.5)
    assert abs(y[2] - math.cos(th)) < 1e-6 and abs(y[3] - math.sin(th)) < 1e-6
    assert abs(y[3] - math.sin(10000.0 ** -0.5)) > 1e-3


def test_rope_llama3_kat(orc):
    # Port of inference/tests.rs:8447 apply_rope_uses_llama3_frequency_scaling_metadata.
    c, s = orc.rope_tables(4, 10000.0, 2, 8.0, 16.0, 1.0, 4.0, None, 8, 1)
    y = orc.apply_rope(np.array([0, 0, 1, 0], np.float32), 1, 4, 4, c[0], s[0])
    base = 10000.0 ** -0.5
    scaled = base / 8.0
    assert abs(y[2] - math.cos(8 * scaled)) < 1e-6
    assert abs(y[3] - math.sin(8 * scaled)) < 1e-6
    assert abs(y[3] - math.sin(8 * base)) > 1e-2


def test_rope_llama3_smooth_band_float64(orc):
    # The smoothing branch against a float64 evaluation of the llama3 formula.
    rd, base, factor, orig, low, high = 128, 500000.0, 32.0, 8192.0, 1.0, 4.0
    c, s = orc.rope_tables(rd, base, 2, factor, orig, low, high, None, 1, 1)
    ang = np.arctan2(s[0].astype(np.float64), c[0].astype(np.float64))
    want = []
    for i in range(rd // 2):
        f = base ** (-2.0 * i / rd)
        wl = 2 * math.pi / f
        if wl < orig / high:
            g = f
        elif wl > orig / low:
            g = f / factor
        else:
            sm = (orig / wl - low) / (high - low)
            g = (1 - sm) * f / factor + sm * f
        want.append(g)
    assert np.allclose(ang, np.array(want), rtol=2e-5, atol=1e-9)


# ------------------------------------------------------------------ KV + attention
def test_kv_f16_rounding_kat(orc):
    # Port of inference/tests.rs:11323 kv_cache_storage_matches_llama_cpp_f16_rounding.
    x = np.array([1.0001, -2.0003, 3.0007, -4.0009], np.float32)
    r = orc.f16_to_f32(orc.f32_to_f16(x))
    assert np.array_equal(r, x.astype(np.float16).astype(np.float32))
    assert not np.array_equal(r, x)


def test_attention_grouped_single_position_kat(orc):
    # Port of inference/tests.rs:11456: one position copies V; heads map grouped (h / repeats).
    kc = np.array([1, 0, 0, 1], np.float32)
    vc = np.array([10, 11, 20, 21], np.float32)
    q = np.array([1, 0, 0, 1, 1, 1, -1, 1], np.float32)
    out = orc.attention(q, kc, vc, 4, 2, 2, 1, 1)
    assert np.array_equal(out, np.array([10, 11, 10, 11, 20, 21, 20, 21], np.float32))


def test_attention_grouped_two_positions_kat(orc):
    # Port of inference/tests.rs:11514 (layout [kv_head][pos][hd]).
    kc = np.array([[1, 0], [0, 1], [0, 1], [1, 0]], np.float32).reshape(2, 2, 2)
    vc = np.array([[10, 0], [0, 11], [20, 0], [0, 21]], np.float32).reshape(2, 2, 2)
    q = np.array([1, 0, 0, 1, 0, 1, 1, 0], np.float32)
    out = orc.attention(q, kc.ravel(), vc.ravel(), 4, 2, 2, 2, 2)
    hi = math.exp(1 / math.sqrt(2))
    ph = hi / (hi + 1)
    pl = 1 - ph
    want = [ph * 10, pl * 11, pl * 10, ph * 11, ph * 20, pl * 21, pl * 20, ph * 21]
    assert np.allclose(out, want, rtol=1e-6)


def test_attention_float64_reference(orc):
    rng = np.random.default_rng(7)
    nh, nkv, hd, P, maxp = 8, 2, 64, 37, 40
    kc = orc.f16_to_f32(orc.f32_to_f16(rng.normal(0, 1, (nkv, maxp, hd)).astype(np.float32)))
    vc = orc.f16_to_f32(orc.f32_to_f16(rng.normal(0, 1, (nkv, maxp, hd)).astype(np.float32)))
    q = rng.normal(0, 1, nh * hd).astype(np.float32)
    out = orc.attention(q, kc.ravel(), vc.ravel(), nh, nkv, hd, maxp, P).reshape(nh, hd)
    for h in range(nh):
        g = h // (nh // nkv)
        sc = kc[g, :P].astype(np.float64) @ q[h * hd:(h + 1) * hd].astype(np.float64) / math.sqrt(hd)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        want = p @ vc[g, :P].astype(np.float64)
        assert np.allclose(out[h], want, rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------ SwiGLU, argmax, expf
def test_silu_mul_closed_form(orc):
    g = np.linspace(-30, 30, 10001).astype(np.float32)
    u = np.linspace(2, -2, 10001).astype(np.float32)
    y = orc.silu_mul(g, u).astype(np.float64)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(y, want, rtol=1e-6, atol=1e-30)
    assert orc.silu_mul(np.zeros(1, np.float32), np.ones(1, np.float32))[0] == 0.0


def test_argmax_brute_force_with_ties(orc):
    rng = np.random.default_rng(8)
    for n in (1, 7, 1000, 32000):
        x = rng.integers(-5, 5, n).astype(np.float32)  # many ties
        assert orc.argmax(x) == int(np.argmax(x))  # numpy returns the first maximum
    assert orc.argmax(np.full(10, -np.inf, np.float32)) == 0


def test_oracle_expf_is_glibc(orc):
    # The oracle calls the platform expf; spot values against float64.
    x = np.linspace(-100, 80, 100001).astype(np.float32)
    y = orc.expf(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    assert np.all(np.abs(y - want) <= 1.0001 * np.spacing(np.float32(want).astype(np.float32)).astype(np.float64) + 1e-45)


# ------------------------------------------------------------------ K-quants (Q8_K, Q4_K, Q6_K)
def test_q4_k_q6_k_dequant_fixtures_match_reference(orc):
    """Q4_K / Q6_K superblock decode vs the reference's gguf==0.19.0 fixtures."""
    for name, quant in (("Q4_K.json", 1), ("Q6_K.json", 2)):
        _, raw, ref = _fixture(name)
        got = orc.dequant_kquant(quant, raw).view(np.uint32)
        assert np.array_equal(got, ref), name


def test_nearest_int_is_round_half_even(orc):
    """nearest_int_reference (inference.rs:17555-17561) == IEEE round-half-even (numpy rint)."""
    xs = np.concatenate([np.arange(-300, 300) + 0.5, np.arange(-300, 300) + 0.25, np.arange(-300, 300) - 0.75,
                         np.random.default_rng(5).uniform(-4e6, 4e6, 2000)]).astype(np.float32)
    got = np.array([orc.nearest_int(v) for v in xs])
    assert np.array_equal(got, np.rint(xs.astype(np.float64)).astype(np.int64))


def test_quantize_q8_k_properties(orc):
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, 256 * 40).astype(np.float32)
    x[256 * 3: 256 * 4] = 0.0                                    # all-zero block
    blk = x[256 * 5: 256 * 6]
    blk[:] = rng.uniform(-1, 1, 256)
    blk[5], blk[9] = -2.0, 2.0                                   # |max| tie: the first (negative) wins
    d, q = orc.quantize_q8_k(x)
    q = q.reshape(-1, 256).astype(np.int64)
    xb = x.reshape(-1, 256)
    assert d[3] == 0.0 and not q[3].any()
    assert q[5, 5] == -127 and q[5, 9] == 127 and d[5] > 0
    for b in range(len(d)):
        if b == 3:
            continue
        i = int(np.argmax(np.abs(xb[b])))
        assert q[b, i] == -127                                   # the max maps to -127 (iscale = -127/max)
        assert np.all(np.abs(q[b]) <= 127)
        err = np.abs(d[b].astype(np.float64) * q[b] - xb[b])
        assert np.all(err <= abs(float(d[b])) * 0.5 * (1 + 1e-5))


def _kquant_exact_case(orc, rng, quant, rows, nsb):
    """Wire bytes with power-of-two scales and small activations: every product and sum of the
    dot is exact in f32, so the dot must equal the float64 sum over the (fixture-pinned)
    dequantized weights."""
    bb = 144 if quant == 1 else 210
    wire = rng.integers(0, 256, (rows, nsb, bb), dtype=np.uint8)
    if quant == 1:
        d = (2.0 ** rng.integers(-6, -4, (rows, nsb, 2))).astype(np.float32)
        wire[:, :, 0:4] = orc.f32_to_f16(d).view(np.uint8).reshape(rows, nsb, 4)
    else:
        d = (2.0 ** rng.integers(-6, -4, (rows, nsb))).astype(np.float32)
        wire[:, :, 208:210] = orc.f32_to_f16(d).view(np.uint8).reshape(rows, nsb, 2)
        wire[:, :, 192:208] = rng.integers(-8, 9, (rows, nsb, 16)).astype(np.int8).view(np.uint8)
    wire = wire.ravel()
    yd = (2.0 ** rng.integers(-1, 1, nsb)).astype(np.float32)
    yq = rng.integers(-3, 4, nsb * 256).astype(np.int8)
    return wire, yd, yq


@pytest.mark.parametrize("quant", [1, 2])
def test_kquant_dot_exact_case_equals_dequant_sum(orc, quant):
    rng = np.random.default_rng(10 + quant)
    rows, nsb = 64, 2
    wire, yd, yq = _kquant_exact_case(orc, rng, quant, rows, nsb)
    got = orc.kquant_gemv(quant, wire, rows, nsb * 256, yd, yq)
    w = orc.dequant_kquant(quant, wire).reshape(rows, nsb * 256).astype(np.float64)
    x = yq.astype(np.float64) * np.repeat(yd.astype(np.float64), 256)
    assert np.array_equal(got.astype(np.float64), (w * x[None, :]).sum(1))


@pytest.mark.parametrize("quant", [1, 2])
def test_kquant_dot_float64_bound(orc, quant):
    """Random superblocks (finite scales): the f32 dot is within a float64 error bound of the
    exact dequantized sum."""
    rng = np.random.default_rng(20 + quant)
    rows, nsb = 128, 8
    bb = 144 if quant == 1 else 210
    wire = rng.integers(0, 256, (rows, nsb, bb), dtype=np.uint8)
    if quant == 1:
        wire[:, :, 0:4] = orc.f32_to_f16(rng.uniform(1e-3, 1e-2, (rows, nsb, 2)).astype(np.float32)).view(
            np.uint8).reshape(rows, nsb, 4)
    else:
        wire[:, :, 208:210] = orc.f32_to_f16(rng.uniform(1e-3, 1e-2, (rows, nsb)).astype(np.float32)).view(
            np.uint8).reshape(rows, nsb, 2)
    wire = wire.ravel()
    yd, yq = orc.quantize_q8_k(rng.normal(0, 1, nsb * 256).astype(np.float32))
    got = orc.kquant_gemv(quant, wire, rows, nsb * 256, yd, yq).astype(np.float64)
    w = orc.dequant_kquant(quant, wire).reshape(rows, nsb * 256).astype(np.float64)
    x = yq.astype(np.float64) * np.repeat(yd.astype(np.float64), 256)
    exact = (w * x[None, :]).sum(1)
    bound = 1e-5 * (np.abs(w) * np.abs(x)[None, :]).sum(1) + 1e-6
    assert np.all(np.abs(got - exact) <= bound)
