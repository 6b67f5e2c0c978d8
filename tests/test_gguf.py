"""The GGUF mapping and parser (include/camelid_gguf.h) on the CPU: the reference's own GGUF
tests (tests/gguf_metadata.rs) and committed fixtures (tests/fixtures/gguf, copied to
tests/golden/gguf with their SHA256SUMS), the malformed-file refusals of
src/gguf/reader.rs:346-470, and a synthetic model's tensors round-tripping byte for byte."""
from __future__ import annotations

import ctypes as C
import hashlib
import struct
from pathlib import Path

import numpy as np
import pytest

from camelid_amd import _native as N
from camelid_amd.model import GgufModel, SyntheticModel, tiny_config
from gguf_writer import ARR, F32, GGML, I32, STR, U32, gguf_bytes, model_gguf

FIX = Path(__file__).resolve().parent / "golden" / "gguf"


def _open(path):
    lib = N.lib()
    h = N.vp()
    rc = lib.camelid_gguf_open(str(path).encode(), C.byref(h))
    return rc, h, (lib.camelid_gguf_last_error().decode() if rc else "")


def _refusal(tmp_path, data: bytes) -> str:
    p = tmp_path / "bad.gguf"
    p.write_bytes(data)
    rc, h, msg = _open(p)
    if rc == 0:
        N.lib().camelid_gguf_close(h)
    assert rc != 0, "the file must be refused"
    return msg


def test_parses_minimal_gguf_like_the_reference(tmp_path):
    """tests/gguf_metadata.rs:6-30: one F32 tensor [4, 2], three metadata keys."""
    data = gguf_bytes([("general.architecture", STR, "llama"), ("general.name", STR, "tiny-test"),
                       ("general.alignment", U32, 32)],
                      [("token_embd.weight", [4, 2], 0, np.arange(8, dtype=np.float32).tobytes())])
    p = tmp_path / "tiny.gguf"
    p.write_bytes(data)
    rc, h, msg = _open(p)
    assert rc == 0, msg
    lib = N.lib()
    try:
        assert lib.camelid_gguf_version(h) == 3 and lib.camelid_gguf_tensor_count(h) == 1
        assert lib.camelid_gguf_meta_str(h, b"general.architecture") == b"llama"
        assert lib.camelid_gguf_meta_str(h, b"general.name") == b"tiny-test"
        assert lib.camelid_gguf_alignment(h) == 32
        t = N.GgufTensor()
        assert lib.camelid_gguf_find(h, b"token_embd.weight", C.byref(t)) == 0
        assert list(t.dims[:t.n_dims]) == [4, 2] and t.type == 0 and t.n_bytes == 32
        assert t.offset % 32 == 0
        got = np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), (8,))
        assert np.array_equal(got, np.arange(8, dtype=np.float32))
        assert lib.camelid_gguf_find(h, b"nope", C.byref(t)) != 0
    finally:
        lib.camelid_gguf_close(h)


def test_refusals(tmp_path):
    """tests/gguf_metadata.rs:32-74 (bad magic, duplicate key, non-contiguous offsets) and the
    other checks of read_metadata_with_len."""
    t1 = [("a.weight", [32], 0, b"\0" * 128)]
    ok_meta = [("general.architecture", STR, "llama")]
    assert "bad magic" in _refusal(tmp_path, b"GGUX" + gguf_bytes(ok_meta, t1)[4:])
    dup = [("general.architecture", STR, "llama"), ("general.architecture", STR, "llama")]
    assert "duplicate metadata key general.architecture" in _refusal(tmp_path, gguf_bytes(dup, t1))
    two = [("a.weight", [32], 0, b"\0" * 128), ("b.weight", [32], 0, b"\0" * 128)]
    msg = _refusal(tmp_path, gguf_bytes(ok_meta, two, offsets=[32, 160]))
    assert "not contiguous" in msg and "expected 0" in msg
    assert "expected v2 or v3" in _refusal(tmp_path, gguf_bytes(ok_meta, t1, version=1))
    assert "invalid alignment 3" in _refusal(tmp_path, gguf_bytes(ok_meta + [("general.alignment", U32, 3)], t1))
    assert "non-integer" in _refusal(tmp_path, gguf_bytes(ok_meta + [("general.alignment", STR, "32")], t1))
    assert "nested" in _refusal(tmp_path, gguf_bytes(ok_meta + [("x", ARR, (ARR, []))], t1))
    full = gguf_bytes(ok_meta, t1)
    assert "beyond end of file" in _refusal(tmp_path, full[:-1])
    assert "end of file" in _refusal(tmp_path, full[:40])
    assert "not divisible by block size 32" in _refusal(tmp_path, gguf_bytes(ok_meta, [("q.weight", [48], 8, b"\0" * 51)]))
    assert "negative tensor or metadata count" in _refusal(tmp_path, b"GGUF" + struct.pack("<Iqq", 3, -1, 0))
    assert "duplicate tensor name a.weight" in _refusal(
        tmp_path, gguf_bytes(ok_meta, [("a.weight", [32], 0, b"\0" * 128), ("a.weight", [32], 0, b"\0" * 128)]))
    assert "empty file" in _refusal(tmp_path, b"")


def _sha256sums():
    out = {}
    for line in (FIX / "SHA256SUMS").read_text().splitlines():
        sha, name = line.split("  ")
        out[name] = sha
    return out


def test_reference_fixtures_are_pinned():
    for name, sha in _sha256sums().items():
        assert hashlib.sha256((FIX / name).read_bytes()).hexdigest() == sha, name


def test_reference_fixture_refusals_and_parses():
    """tests/invariant_matrix_binding.rs:564-640, tests/nvfp4_wire_lane_refusals.rs:62-111:
    an unknown GGML type (41) and an NVFP4 tensor with K % 64 != 0 refuse at parse, naming the
    tensor; the four other fixtures parse (architecture gemma4)."""
    rc, _, msg = _open(FIX / "nvfp4_unknown_type_trip.gguf")
    assert rc and "blk.0.mystery.weight" in msg and "41" in msg
    rc, _, msg = _open(FIX / "nvfp4_k_div_trip.gguf")
    assert rc and "first dimension 48 is not divisible by block size 64" in msg and "blk.0.ffn_down.weight" in msg
    lib = N.lib()
    sidecar = ["blk.0.ffn_down.weight", "blk.0.ffn_down.weight.scale", "blk.0.ffn_down.weight.input_scale"]
    for name, tensors in (("nvfp4_sidecar_admit_trip.gguf", sidecar), ("nvfp4_sidecar_trip.gguf", sidecar),
                          ("nvfp4_pilot_admit.gguf", ["blk.0.ffn_down.weight"]),
                          ("nvfp4_nan_sentinel_trip.gguf", ["blk.0.ffn_up.weight"])):
        rc, h, msg = _open(FIX / name)
        assert rc == 0, (name, msg)
        assert lib.camelid_gguf_meta_str(h, b"general.architecture") == b"gemma4"
        # the resident path's model reader refuses the architecture (not on this path)
        dims, rope = N.Dims(), N.GgufRope()
        assert lib.camelid_gguf_model(h, 64, C.byref(dims), C.byref(rope)) != 0
        assert [lib.camelid_gguf_tensor_name(h, i).decode() for i in range(lib.camelid_gguf_tensor_count(h))] == tensors
        t = N.GgufTensor()
        assert lib.camelid_gguf_find(h, tensors[0].encode(), C.byref(t)) == 0
        assert t.type == 40 and list(t.dims[:t.n_dims]) == [64] and t.n_bytes == 36  # NVFP4: 64 values, 36 bytes
        for side in tensors[1:]:
            assert lib.camelid_gguf_find(h, side.encode(), C.byref(t)) == 0 and t.type == 0 and t.n_bytes == 4
        lib.camelid_gguf_close(h)


@pytest.mark.parametrize("kw,arch", [(dict(), "llama"),
                                     (dict(tied=True, rope_scaling="llama3", rope_factor=32.0, rope_theta=500000.0),
                                      "llama"),
                                     (dict(hidden=512, ffn_dim=768, n_heads=4, n_kv_heads=2, head_dim=128, vocab=1024,
                                           qk_norm=True, split_half=True, rope_theta=1e6, eps=1e-6,
                                           quant_scheme="q4_k_m"), "qwen3")])
def test_model_round_trip(tmp_path, kw, arch):
    """A synthetic model written as GGUF: the config read back equals the model's, every
    tensor's mapped bytes equal the written ones, the embedding rows and RoPE tables equal
    the synthetic model's."""
    cfg = tiny_config(**kw)
    model = SyntheticModel.generate(cfg)
    p = tmp_path / "m.gguf"
    p.write_bytes(model_gguf(model, arch, alignment=64))
    g = GgufModel(p, 128)
    try:
        c = g.cfg
        for f in ("n_layers", "hidden", "ffn_dim", "n_heads", "n_kv_heads", "head_dim", "vocab", "tied", "qk_norm",
                  "split_half", "rope_scaling"):
            assert getattr(c, f) == getattr(cfg, f), f
        for f in ("rope_theta", "eps", "rope_factor"):
            assert np.float32(getattr(c, f)) == np.float32(getattr(cfg, f)), f
        assert np.array_equal(g.tensor_bytes("blk.1.ffn_down.weight"), model.layers[1]["projs"]["down"])
        assert np.array_equal(g.tensor_bytes("token_embd.weight"), model.token_embd)
        toks = [0, 5, cfg.vocab - 1]
        assert np.array_equal(g.embed(toks), model.embed(toks))
        for a, b in zip(g.rope_tables(3, 9), model.rope_tables(3, 9)):
            assert np.array_equal(a, b)
        assert N.lib().camelid_gguf_alignment(g._h) == 64
    finally:
        g.close()


def test_element_count_overflow_is_refused(tmp_path):
    """reader.rs:553-557 (checked_mul of the dims): a tensor whose element count passes 2^64
    is refused, not wrapped to a small byte count."""
    ok_meta = [("general.architecture", STR, "llama")]
    msg = _refusal(tmp_path, gguf_bytes(ok_meta, [("a.weight", [2 ** 32, 2 ** 32, 2 ** 32, 2 ** 32], 0, b"")]))
    assert "element count overflows" in msg
    msg = _refusal(tmp_path, gguf_bytes(ok_meta, [("a.weight", [2 ** 32, 2 ** 32], 0, b"")]))
    assert "element count overflows" in msg
    # just below 2^64 elements: not an overflow, but far beyond the file
    assert "beyond end of file" in _refusal(tmp_path, gguf_bytes(ok_meta, [("a.weight", [2 ** 32, 2 ** 31], 0, b"")]))


def _model_with_rope_freqs(tmp_path, dims, ggml_type, data):
    cfg = tiny_config()
    model = SyntheticModel.generate(cfg)
    p = tmp_path / "rf.gguf"
    p.write_bytes(model_gguf(model, "llama", extra_tensors=[("rope_freqs.weight", dims, ggml_type, data)]))
    rc, h, msg = _open(p)
    assert rc == 0, msg
    lib = N.lib()
    d, rope = N.Dims(), N.GgufRope()
    rc = lib.camelid_gguf_model(h, 64, C.byref(d), C.byref(rope))
    msg = lib.camelid_gguf_last_error().decode() if rc else ""
    got = None
    if rc == 0 and rope.freqs:
        got = np.ctypeslib.as_array(C.cast(rope.freqs, C.POINTER(C.c_float)), (cfg.rope_dim // 2,)).copy()
    lib.camelid_gguf_close(h)
    return rc, msg, got


def test_rope_freqs_shape_type_and_values_are_validated(tmp_path):
    """model.rs:938-944 require_descriptor_shape(rope_freqs, [rope_dim/2]) and rope.rs:287-312
    validate_rope_frequency_tensor: any other descriptor shape ([half, 0], [half, 2], a short
    [half - 1]) and any factor that is not finite and positive refuse the model, with the
    reference's reason; F32 is read in place, F16 and BF16 widened as load_cpu_f32 does
    (tensor/mod.rs:3943-3946)."""
    half = tiny_config().rope_dim // 2
    for dims in ([half, 0], [half, 2], [half - 1]):
        n = int(np.prod(dims))
        rc, msg, _ = _model_with_rope_freqs(tmp_path, dims, 0, np.full(n, 2.0, np.float32).tobytes())
        assert rc != 0 and "expected descriptor shape" in msg, (dims, msg)
    for bad in (0.0, -1.0, np.inf, np.nan):
        vals = np.full(half, 2.0, np.float32)
        vals[3] = bad
        rc, msg, _ = _model_with_rope_freqs(tmp_path, [half], 0, vals.tobytes())
        assert rc != 0 and "rope_freqs.weight[3]" in msg and "finite and positive" in msg, (bad, msg)
    vals = np.linspace(0.5, 8.0, half, dtype=np.float32)
    rc, msg, got = _model_with_rope_freqs(tmp_path, [half], 0, vals.tobytes())
    assert rc == 0, msg
    assert np.array_equal(got, vals)
    # F16 and BF16 (subnormal and normal halves; every half is exact in f32)
    h16 = np.array([2.0 ** -20, 6.1e-5, 0.5, 1.0, 1.5, 3.140625, 1000.0, 65504.0] * (half // 8 + 1), np.float16)[:half]
    rc, msg, got = _model_with_rope_freqs(tmp_path, [half], 1, h16.tobytes())
    assert rc == 0, msg
    assert np.array_equal(got, h16.astype(np.float32))
    b16 = (vals.view(np.uint32) >> 16).astype(np.uint16)
    rc, msg, got = _model_with_rope_freqs(tmp_path, [half], 30, b16.tobytes())
    assert rc == 0, msg
    assert np.array_equal(got, (b16.astype(np.uint32) << 16).view(np.float32))
