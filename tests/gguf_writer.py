"""GGUF v3 writer for the tests: a synthetic model (or hand-built pieces of one) as a file the
native loader maps.  Layout per the format the reference parses (src/gguf/reader.rs:346-470):
magic, version, i64 counts, typed metadata, tensor infos (name, dims, GGML type, offset
relative to the aligned data start), then the tensor data at the alignment."""
from __future__ import annotations

import struct

import numpy as np

from camelid_amd.engine import Q4_K, Q6_K, Q8_0

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
GGML = {Q8_0: 8, Q4_K: 12, Q6_K: 14, "f32": 0}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(ty: int, v) -> bytes:
    if ty == STR:
        return _str(v)
    if ty == ARR:
        ety, items = v
        return struct.pack("<iQ", ety, len(items)) + b"".join(_value(ety, x) for x in items)
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}[ty]
    return struct.pack(fmt, v)


def gguf_bytes(meta: list, tensors: list, alignment: int = 32, version: int = 3,
               offsets: list | None = None) -> bytes:
    """meta: [(key, type, value)]; tensors: [(name, dims, ggml_type, data bytes)].  offsets
    overrides the relative offsets written (to build malformed files)."""
    out = bytearray(b"GGUF" + struct.pack("<Iqq", version, len(tensors), len(meta)))
    for key, ty, v in meta:
        out += _str(key) + struct.pack("<i", ty) + _value(ty, v)
    rel, pos = [], 0
    for _, _, _, data in tensors:
        rel.append(pos)
        pos = (pos + len(data) + alignment - 1) // alignment * alignment
    if offsets is not None:
        rel = offsets
    for (name, dims, ty, _), off in zip(tensors, rel):
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<q", d) for d in dims)
        out += struct.pack("<iQ", ty, off)
    out += b"\0" * ((-len(out)) % alignment)
    start = len(out)
    for (_, _, _, data), off in zip(tensors, rel):
        need = start + off - len(out)
        if need > 0:
            out += b"\0" * need
        out += bytes(data)
    return bytes(out)


def model_gguf(model, arch: str = "llama", alignment: int = 32, extra_meta: list | None = None,
               extra_tensors: list | None = None) -> bytes:
    """A SyntheticModel as a GGUF file: the GGUF tensor names, weights as their wire bytes,
    norms as F32, dims [k, rows] (the contiguous dimension first); extra_tensors are appended
    as given ([(name, dims, ggml_type, data bytes)])."""
    cfg = model.cfg
    a = arch
    meta = [("general.architecture", STR, a), ("general.name", STR, cfg.name), ("general.alignment", U32, alignment),
            (f"{a}.block_count", U32, cfg.n_layers), (f"{a}.context_length", U32, 4096),
            (f"{a}.embedding_length", U32, cfg.hidden), (f"{a}.feed_forward_length", U32, cfg.ffn_dim),
            (f"{a}.attention.head_count", U32, cfg.n_heads), (f"{a}.attention.head_count_kv", U32, cfg.n_kv_heads),
            (f"{a}.attention.key_length", U32, cfg.head_dim), (f"{a}.rope.dimension_count", U32, cfg.rope_dim),
            (f"{a}.attention.layer_norm_rms_epsilon", F32, cfg.eps), (f"{a}.rope.freq_base", F32, cfg.rope_theta),
            ("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(8)])),
            ("tokenizer.ggml.scores", ARR, (F32, [0.0] * 8))]
    if cfg.rope_scaling != "none":
        meta += [(f"{a}.rope.scaling.type", STR, cfg.rope_scaling), (f"{a}.rope.scaling.factor", F32, cfg.rope_factor)]
        if cfg.rope_scaling == "llama3":
            meta += [(f"{a}.rope.scaling.original_context_length", U32, int(cfg.rope_orig_ctx)),
                     (f"{a}.rope.scaling.low_freq_factor", F32, cfg.rope_low),
                     (f"{a}.rope.scaling.high_freq_factor", F32, cfg.rope_high)]
    meta += extra_meta or []
    H = cfg.hidden
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate", "up": "ffn_up",
             "down": "ffn_down"}
    shapes = cfg.proj_shapes()
    f32 = lambda x: np.ascontiguousarray(x, np.float32).tobytes()
    tensors = [("token_embd.weight", [H, cfg.vocab], GGML[cfg.embd_quant()], model.token_embd.tobytes())]
    for i, L in enumerate(model.layers):
        p = f"blk.{i}."
        tensors.append((p + "attn_norm.weight", [H], 0, f32(L["attn_norm"])))
        for j, (proj, gname) in enumerate(names.items()):
            rows, k = shapes[proj]
            tensors.append((p + gname + ".weight", [k, rows], GGML[L["quant"][j]], L["projs"][proj].tobytes()))
        tensors.append((p + "ffn_norm.weight", [H], 0, f32(L["ffn_norm"])))
        if "q_norm" in L:
            tensors.append((p + "attn_q_norm.weight", [cfg.head_dim], 0, f32(L["q_norm"])))
            tensors.append((p + "attn_k_norm.weight", [cfg.head_dim], 0, f32(L["k_norm"])))
    tensors.append(("output_norm.weight", [H], 0, f32(model.output_norm)))
    if model.output is not model.token_embd:
        tensors.append(("output.weight", [H, cfg.vocab], GGML[cfg.output_quant()], model.output.tobytes()))
    tensors += extra_tensors or []
    return gguf_bytes(meta, tensors, alignment)
