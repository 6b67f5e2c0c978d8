"""CPU-only checks of the native library: exported C ABI, host seam, expf restatement,
synthetic generator.  No GPU compute is called here."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared_symbols():
    syms = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        syms.update(re.findall(r"\b(camelid_\w+)\s*\(", text))
    return sorted(syms)


def test_library_exports_every_declared_symbol(native):
    from camelid_amd import _native as N
    syms = _declared_symbols()
    assert len(syms) > 30
    out = subprocess.run(["nm", "-D", "--defined-only", str(N.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (camelid_\w+)", out))
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    for s in syms:
        getattr(native, s)  # resolvable through ctypes
    # every declared entry point has a ctypes signature
    assert not [s for s in syms if s not in N.SIGNATURES]


def test_engine_rejects_bad_dims_without_gpu(native):
    from camelid_amd.engine import EngineDims, HipResidentDecode
    from camelid_amd._native import HipError
    with pytest.raises(HipError, match="nonzero|multiple"):
        HipResidentDecode(EngineDims(0, 4, 2, 64, 256, 512, 64, 16, 100, 1e-5))
    with pytest.raises(HipError, match="multiple"):
        HipResidentDecode(EngineDims(1, 5, 2, 64, 256, 512, 64, 16, 100, 1e-5))


def test_expf_restatement_matches_glibc_sampled(native, orc):
    """The product's expf restatement (host build) against the platform glibc expf.
    Dense over the softmax/SiLU range and strided over all 2^32 bit patterns; the two
    known double-rounding-sensitive inputs of glibc's algorithm are included."""
    rng = np.random.default_rng(0)
    strided = (np.arange(0, 2**32, 97, dtype=np.uint64)[: 40_000_000 // 4]).astype(np.uint32).view(np.float32)
    dense = np.linspace(-104.0, 89.0, 4_000_001, dtype=np.float32)
    hx = float.fromhex
    special = np.array([hx("0x1.04845ep+5"), hx("-0x1.f8cbb2p+5"), hx("-0x1.9424fcp-14"), hx("0x1.fefe02p-16"),
                        88.0, -88.0, hx("0x1.62e42ep6"), hx("0x1.62e430p6"), hx("-0x1.9fe368p6"),
                        hx("-0x1.9fe36ap6"), -103.0, 0.0, -0.0, np.inf, -np.inf, 1e-30, -1e-30], np.float32)
    x = np.concatenate([strided, dense, special, rng.normal(0, 10, 1_000_000).astype(np.float32)])
    x = np.ascontiguousarray(x[~np.isnan(x)])
    want = orc.expf(x)
    got = np.empty_like(x)
    from camelid_amd._native import ptr
    native.camelid_expf_host(ptr(x, C.c_float), ptr(got, C.c_float), x.size)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, [(float(x[i]).hex(), float(got[i]).hex(), float(want[i]).hex()) for i in bad[:5]]


def test_seam_rope_tables_match_oracle(native, orc):
    from camelid_amd.model import CONFIGS, rope_tables
    for cfg in (CONFIGS["llama-3.2-3b"], CONFIGS["tinyllama-1.1b"], CONFIGS["mistral-7b-v0.3"]):
        c, s = rope_tables(cfg, 0, 600)
        kind = {"none": 0, "linear": 1, "llama3": 2}[cfg.rope_scaling]
        oc, os_ = orc.rope_tables(cfg.rope_dim, cfg.rope_theta, kind, cfg.rope_factor, cfg.rope_orig_ctx,
                                  cfg.rope_low, cfg.rope_high, None, 0, 600)
        assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
        assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))
        # tables starting at an offset equal the slice of the full table
        c2, s2 = rope_tables(cfg, 123, 5)
        assert np.array_equal(c2, c[123:128]) and np.array_equal(s2, s[123:128])


def test_seam_embedding_and_synth(native, orc):
    from camelid_amd.model import tiny_config, SyntheticModel, prompt_tokens, synth_f32
    cfg = tiny_config()
    m = SyntheticModel.generate(cfg)
    toks = prompt_tokens(cfg)
    assert toks.max() < cfg.vocab and len(toks) == cfg.prompt_len
    emb = m.embed(toks)
    want = orc.dequant_q8_0_wire(m.token_embd).reshape(cfg.vocab, cfg.hidden)[toks]
    assert np.array_equal(emb, want)
    # determinism and distribution of the generator
    m2 = SyntheticModel.generate(cfg)
    assert np.array_equal(m.layers[1]["projs"]["down"], m2.layers[1]["projs"]["down"])
    v = synth_f32("blk.0.attn_q.weight", 3, 1_000_000, 0.02)
    assert abs(v.mean()) < 1e-4 and abs(v.std() - 0.02) < 1e-4
    # the Q8_0 stream is the quantized f32 stream
    w = synth_f32("blk.0.attn_q.weight", cfg.seed, cfg.nq * cfg.hidden, cfg.weight_std)
    assert np.array_equal(orc.quantize_q8_0_wire(w), m.layers[0]["projs"]["q"])


def test_q8_repack_layouts(native, orc):
    from camelid_amd._native import ptr
    rng = np.random.default_rng(3)
    rows, k = 17, 96
    wire = orc.quantize_q8_0_wire(rng.normal(0, 0.02, rows * k).astype(np.float32))
    q = np.empty(rows * k, np.int8)
    d = np.empty(rows * k // 32, np.uint16)
    assert native.camelid_q8_0_repack(ptr(wire, C.c_uint8), rows, k, 34, ptr(q, C.c_int8), ptr(d, C.c_uint16)) == 0
    blocks = wire.reshape(-1, 34)
    assert np.array_equal(d, blocks[:, :2].copy().view(np.uint16).ravel())
    assert np.array_equal(q.reshape(-1, 32), blocks[:, 2:].view(np.int8))
    # 36-byte Q8_0Block layout (f32 scale) repacks to the same planes
    b36 = np.zeros((rows * k // 32, 36), np.uint8)
    b36[:, :4] = orc.f16_to_f32(d).view(np.uint8).reshape(-1, 4)
    b36[:, 4:] = blocks[:, 2:]
    q2 = np.empty_like(q)
    d2 = np.empty_like(d)
    assert native.camelid_q8_0_repack(ptr(b36.ravel(), C.c_uint8), rows, k, 36, ptr(q2, C.c_int8),
                                      ptr(d2, C.c_uint16)) == 0
    assert np.array_equal(q, q2) and np.array_equal(d, d2)


def test_check_model_refuses_unsupported_shapes_without_gpu(native):
    """camelid_hip_check_model: the host preflight of the resident engine's decline
    (build_resident_cuda_engine returns None, inference.rs:11245).  K-quant rows wider than the
    GEMV kernels take (ffn_down of a Q4_K qwen2-7B, ffn 18944) are refused with a reason, as are
    rows whose width is no multiple of the block; the benchmark configs are taken."""
    from camelid_amd import _native as N
    from camelid_amd.engine import Q4_K, Q6_K, Q8_0
    from camelid_amd.model import CONFIGS

    def check(dims, quant, out):
        q = (C.c_uint8 * 7)(*quant) if quant is not None else None
        rc = native.camelid_hip_check_model(C.byref(dims), C.cast(q, N.u8p) if q is not None else None, out)
        return rc, N.last_error()

    def dims_of(cfg, max_pos=2048, **over):
        d = N.Dims(cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.hidden, cfg.ffn_dim, cfg.rope_dim,
                   max_pos, cfg.vocab, cfg.eps, int(cfg.split_half))
        for k, v in over.items():
            setattr(d, k, v)
        return d

    q8 = [Q8_0] * 7
    qkm = [Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, Q4_K]
    for name, cfg in CONFIGS.items():
        quant = q8 if cfg.quant_scheme == "q8_0" else qkm
        out = Q8_0 if cfg.quant_scheme == "q8_0" else Q6_K
        assert check(dims_of(cfg, cfg.prompt_len + cfg.decode_len), quant, out)[0] == 0, name
    qwen = CONFIGS["qwen3-8b"]
    rc, msg = check(dims_of(qwen, ffn_dim=18944), qkm, Q6_K)
    assert rc != 0 and "down projection" in msg and "18944 > 16384" in msg
    # the same width in Q8_0 is taken (its GEMV stages the row in LDS up to the limit checked here)
    assert check(dims_of(qwen, ffn_dim=18944), [Q4_K] * 6 + [Q8_0], Q6_K)[0] == 0
    rc, msg = check(dims_of(qwen, hidden=4096 + 32), qkm, Q6_K)
    assert rc != 0 and "multiple of 256" in msg
    rc, msg = check(dims_of(qwen), qkm, 7)
    assert rc != 0 and "output projection" in msg
    assert check(dims_of(qwen), None, Q8_0)[0] == 0
    rc, msg = check(dims_of(qwen, n_kv_heads=3), None, Q8_0)
    assert rc != 0 and "multiple of n_kv_heads" in msg


def test_engine_wrapper_refuses_short_arrays_without_gpu(native):
    """The Python mirror checks every host array against the model dims before the C side
    copies its fixed sizes (cuda_resident.rs:7795 checks prefill's lengths the same way):
    short or mis-shaped arrays raise ValueError and no native call is made."""
    from camelid_amd.engine import EngineDims, HipResidentDecode
    d = EngineDims(2, 4, 2, 64, 256, 512, 64, 32, 100, 1e-5)
    eng = object.__new__(HipResidentDecode)  # no device: only the host-side checks run
    eng.dims, eng._lib, eng._h = d, None, None
    H, half = d.hidden, d.rope_dim // 2
    z = np.zeros
    with pytest.raises(ValueError, match="embedding"):
        eng.forward_token(z(H - 1), z(half), z(half), 0, 0.125)
    with pytest.raises(ValueError, match="cos"):
        eng.forward_token(z(H), z(half - 1), z(half), 0, 0.125)
    with pytest.raises(ValueError, match="sin"):
        eng.forward_token(z(H), z(half), z(half + 1), 0, 0.125)
    with pytest.raises(ValueError, match="embeddings"):
        eng.prefill(z((3, H - 32)), z((3, half)), z((3, half)), 0.125)
    with pytest.raises(ValueError, match="rows"):
        eng.prefill(z((3, H)), z((2, half)), z((3, half)), 0.125)
    with pytest.raises(ValueError, match="rows"):
        eng.verify_batch(z((4, H)), z((4, half)), z((3, half)), 0, 0.125)
    with pytest.raises(ValueError, match="cos_all"):
        eng.set_rope_table(z((8, half + 1)), z((8, half + 1)))
    with pytest.raises(ValueError, match="ck"):
        eng.seed_layer(0, z(d.n_kv_heads * 5 * d.head_dim - 1), z(d.n_kv_heads * 5 * d.head_dim), 5)
    with pytest.raises(ValueError, match="final_norm"):
        eng.set_output(z(H + 1), z(10, np.uint8))
    projs = {n: z(8, np.uint8) for n in ("q", "k", "v", "o", "gate", "up", "down")}
    with pytest.raises(ValueError, match="attn_norm"):
        eng.set_layer(0, projs, z(H - 1), z(H))
    with pytest.raises(ValueError, match="k_norm"):
        eng.set_layer(0, projs, z(H), z(H), z(d.head_dim), z(d.head_dim - 1))
