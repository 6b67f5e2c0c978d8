"""Model configurations, seeded synthetic GGUF-style weights, and the greedy session.

The session mirrors Camelid's generation loop over the resident seam
(inference.rs:4383-4425): the first n-1 prompt tokens are prefilled, the last prompt
token runs as a decode step that yields the first generated token, and each later step
feeds the previous greedy token back.  Embedding rows and RoPE tables are computed on the
host, as the seam does (inference.rs:2667-2670, rope.rs:568-627).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import _native as N
from .engine import EngineDims, HipResidentDecode, PROJ_NAMES, Q4_K, Q6_K, Q8_0

Q8_BLOCK_BYTES = 34
# bytes per value of each weight format (Q8_0 34 B / 32, Q4_K 144 B / 256, Q6_K 210 B / 256)
QUANT_BYTES = {Q8_0: 34 / 32, Q4_K: 144 / 256, Q6_K: 210 / 256}


@dataclass(frozen=True)
class ModelConfig:
    name: str
    n_layers: int
    hidden: int
    ffn_dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    vocab: int
    rope_theta: float
    eps: float = 1e-5
    tied: bool = False
    qk_norm: bool = False
    split_half: bool = False
    rope_scaling: str = "none"            # none | linear | llama3
    rope_factor: float = 1.0
    rope_orig_ctx: float = 8192.0
    rope_low: float = 1.0
    rope_high: float = 4.0
    seed: int = 0
    prompt_seed: int = 1
    prompt_len: int = 128
    decode_len: int = 128
    weight_std: float = 0.02
    # "q8_0": every tensor Q8_0.  "q4_k_m": Q4_K for q, k, o, gate, up, down and the token
    # table; Q6_K for v and the output projection (the llama.cpp Q4_K_M mix).
    quant_scheme: str = "q8_0"

    def proj_quant(self, proj: str) -> int:
        if self.quant_scheme == "q8_0":
            return Q8_0
        return Q6_K if proj == "v" else Q4_K

    def output_quant(self) -> int:
        return Q8_0 if self.quant_scheme == "q8_0" else Q6_K

    def embd_quant(self) -> int:
        return Q8_0 if self.quant_scheme == "q8_0" else Q4_K

    @property
    def rope_dim(self) -> int:
        return self.head_dim

    @property
    def nq(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def nkv(self) -> int:
        return self.n_kv_heads * self.head_dim

    def proj_shapes(self) -> dict:
        """(rows, k) of every projection: GGUF [in, out] stored out-major (inference.rs:2172-2176)."""
        H, F = self.hidden, self.ffn_dim
        return {"q": (self.nq, H), "k": (self.nkv, H), "v": (self.nkv, H), "o": (H, self.nq),
                "gate": (F, H), "up": (F, H), "down": (H, F)}

    def weight_bytes(self) -> int:
        """Weight + norm bytes touched per decode token (lm_head + norms, no embedding)."""
        per_layer = sum(int(r * k * QUANT_BYTES[self.proj_quant(p)]) for p, (r, k) in self.proj_shapes().items())
        norms = 4 * (2 * self.n_layers + 1) * self.hidden
        if self.qk_norm:
            norms += 4 * 2 * self.n_layers * self.head_dim
        lm = int(self.vocab * self.hidden * QUANT_BYTES[self.output_quant()])
        return per_layer * self.n_layers + norms + lm

    def kv_bytes_per_pos(self) -> int:
        return 2 * self.n_layers * self.nkv * 2

    def decode_bytes(self, pos: int) -> int:
        """Algorithmic HBM bytes of one decode step at position `pos` (reads pos+1 KV rows)."""
        emb = int(self.hidden * QUANT_BYTES[self.embd_quant()])
        return self.weight_bytes() + emb + self.kv_bytes_per_pos() * (pos + 1) + self.kv_bytes_per_pos()

    def engine_dims(self, max_pos: int | None = None) -> EngineDims:
        return EngineDims(self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim, self.hidden, self.ffn_dim,
                          self.rope_dim, max_pos or (self.prompt_len + self.decode_len), self.vocab, self.eps,
                          self.split_half)

    def scale(self) -> float:
        # diagnostic_config.rs:300-305: 1 / sqrt(head_dim) in f32
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_dim)))

    def scaled(self, **kw) -> "ModelConfig":
        d = dict(self.__dict__)
        d.update(kw)
        return ModelConfig(**d)


CONFIGS = {
    # TinyLlama-1.1B architecture, seed 0, prompt seed 1, 128 + 128.
    "tinyllama-1.1b": ModelConfig("tinyllama-1.1b", 22, 2048, 5632, 32, 4, 64, 32000, 10000.0,
                                  seed=0, prompt_seed=1, prompt_len=128, decode_len=128),
    # Llama-3.2-3B architecture, tied embeddings, llama3 RoPE scaling, 512 + 256.
    "llama-3.2-3b": ModelConfig("llama-3.2-3b", 28, 3072, 8192, 24, 8, 128, 128256, 500000.0, tied=True,
                                rope_scaling="llama3", rope_factor=32.0, rope_orig_ctx=8192.0, rope_low=1.0,
                                rope_high=4.0, seed=3, prompt_seed=3 + 1000, prompt_len=512, decode_len=256),
    # Mistral-7B-v0.3 architecture, long context 8192 + 256.
    "mistral-7b-v0.3": ModelConfig("mistral-7b-v0.3", 32, 4096, 14336, 32, 8, 128, 32768, 1e6, seed=4,
                                   prompt_seed=4 + 1000, prompt_len=8192, decode_len=256),
    # Qwen3-8B architecture, Q4_K_M (Q6_K v / output), QK-norm, split-half RoPE.
    "qwen3-8b": ModelConfig("qwen3-8b", 36, 4096, 12288, 32, 8, 128, 151936, 1e6, eps=1e-6, qk_norm=True,
                            split_half=True, seed=5, prompt_seed=5 + 1000, prompt_len=1024, decode_len=256,
                            quant_scheme="q4_k_m"),
}


def rope_tables(cfg: ModelConfig, pos0: int, n_pos: int, freqs: np.ndarray | None = None):
    """Host RoPE tables [n_pos][rope_dim/2] (rope.rs:568-685), via the native seam; freqs: a
    model's rope_freqs factors [rope_dim/2] (rope.rs:526-560), if it has them."""
    half = cfg.rope_dim // 2
    cos = np.empty((n_pos, half), np.float32)
    sin = np.empty((n_pos, half), np.float32)
    kind = {"none": 0, "linear": 1, "llama3": 2}[cfg.rope_scaling]
    fp = None if freqs is None else N.ptr(np.ascontiguousarray(freqs, np.float32), C.c_float)
    rc = N.lib().camelid_rope_tables(cfg.rope_dim, cfg.rope_theta, kind, cfg.rope_factor, cfg.rope_orig_ctx,
                                     cfg.rope_low, cfg.rope_high, fp, pos0, n_pos, N.ptr(cos, C.c_float),
                                     N.ptr(sin, C.c_float))
    if rc:
        raise ValueError("invalid RoPE metadata")
    return cos, sin


def prompt_tokens(cfg: ModelConfig, n: int | None = None) -> np.ndarray:
    n = cfg.prompt_len if n is None else n
    out = np.empty(n, np.uint32)
    N.lib().camelid_synth_tokens(cfg.prompt_seed, cfg.vocab, n, N.ptr(out, C.c_uint32))
    return out


def synth_q8_0(name: str, seed: int, rows: int, k: int, std: float = 0.02) -> np.ndarray:
    out = np.empty(rows * k // 32 * Q8_BLOCK_BYTES, np.uint8)
    rc = N.lib().camelid_synth_q8_0_wire(name.encode(), seed, std, rows * k, N.ptr(out, C.c_uint8))
    if rc:
        raise ValueError("Q8_0 tensor size must be a multiple of 32")
    return out


def synth_kquant(name: str, seed: int, rows: int, k: int, quant: int, std: float = 0.02) -> np.ndarray:
    """N(0, std) weights [rows][k] as Q4_K / Q6_K wire superblocks."""
    out = np.empty(int(rows * k * QUANT_BYTES[quant]), np.uint8)
    rc = N.lib().camelid_synth_kquant_wire(name.encode(), seed, std, rows * k, quant, N.ptr(out, C.c_uint8))
    if rc:
        raise ValueError("K-quant tensor size must be a multiple of 256")
    return out


def synth_weight(name: str, seed: int, rows: int, k: int, quant: int, std: float = 0.02) -> np.ndarray:
    return synth_q8_0(name, seed, rows, k, std) if quant == Q8_0 else synth_kquant(name, seed, rows, k, quant, std)


def synth_f32(name: str, seed: int, n: int, std: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    N.lib().camelid_synth_normal_f32(name.encode(), seed, std, N.ptr(out, C.c_float), n)
    return out


@dataclass
class SyntheticModel:
    """Seeded N(0, std) weights as GGUF wire bytes (Q8_0, or the config's K-quant mix); norms = 1.0."""

    cfg: ModelConfig
    layers: list = field(default_factory=list)
    token_embd: np.ndarray | None = None
    output: np.ndarray | None = None
    output_norm: np.ndarray | None = None

    @classmethod
    def generate(cls, cfg: ModelConfig) -> "SyntheticModel":
        m = cls(cfg)
        H = cfg.hidden
        gguf = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
                "up": "ffn_up", "down": "ffn_down"}
        for i in range(cfg.n_layers):
            projs = {p: synth_weight(f"blk.{i}.{gguf[p]}.weight", cfg.seed, r, k, cfg.proj_quant(p), cfg.weight_std)
                     for p, (r, k) in cfg.proj_shapes().items()}
            layer = {"projs": projs, "attn_norm": np.ones(H, np.float32), "ffn_norm": np.ones(H, np.float32),
                     "quant": [cfg.proj_quant(p) for p in PROJ_NAMES]}
            if cfg.qk_norm:
                layer["q_norm"] = np.ones(cfg.head_dim, np.float32)
                layer["k_norm"] = np.ones(cfg.head_dim, np.float32)
            m.layers.append(layer)
        m.token_embd = synth_weight("token_embd.weight", cfg.seed, cfg.vocab, H, cfg.embd_quant(), cfg.weight_std)
        if cfg.tied and cfg.embd_quant() == cfg.output_quant():
            m.output = m.token_embd
        else:
            m.output = synth_weight("output.weight", cfg.seed, cfg.vocab, H, cfg.output_quant(), cfg.weight_std)
        m.output_norm = np.ones(H, np.float32)
        return m

    def embed(self, tokens) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty((len(toks), self.cfg.hidden), np.float32)
        q = self.cfg.embd_quant()
        if q == Q8_0:
            rc = N.lib().camelid_embed_q8_0(N.ptr(self.token_embd, C.c_uint8), self.cfg.vocab, self.cfg.hidden,
                                            N.ptr(toks, C.c_uint32), len(toks), N.ptr(out, C.c_float))
        else:
            rc = N.lib().camelid_embed_kquant(q, N.ptr(self.token_embd, C.c_uint8), self.cfg.vocab, self.cfg.hidden,
                                              N.ptr(toks, C.c_uint32), len(toks), N.ptr(out, C.c_float))
        if rc:
            raise ValueError("token id out of range")
        return out

    def rope_tables(self, pos0: int, n_pos: int):
        return rope_tables(self.cfg, pos0, n_pos)

    def load_into(self, eng: HipResidentDecode, device_embedding: bool = False) -> None:
        for i, L in enumerate(self.layers):
            eng.set_layer(i, L["projs"], L["attn_norm"], L["ffn_norm"], L.get("q_norm"), L.get("k_norm"),
                          quants=L.get("quant"))
        eng.set_output(self.output_norm, self.output, quant=self.cfg.output_quant())
        if device_embedding:
            eng.set_embedding(self.token_embd, quant=self.cfg.embd_quant())


GGML_TO_QUANT = {8: Q8_0, 12: Q4_K, 14: Q6_K}


class GgufModel:
    """A GGUF model file, mapped read-only by the native loader (camelid_gguf_open:
    GgufWireMmap::map, wire_mmap.rs:78, and read_metadata, gguf/reader.rs:346): its config
    (ModelConfig::from_gguf, model.rs:137-230), the seam's embedding rows read from the
    mapped token table, and the upload of every tensor straight from the mapping
    (camelid_hip_load_gguf).  Same interface as SyntheticModel."""

    def __init__(self, path, max_pos: int = 0):
        lib = N.lib()
        self._lib = lib
        h = N.vp()
        if lib.camelid_gguf_open(str(path).encode(), C.byref(h)):
            raise ValueError(lib.camelid_gguf_last_error().decode())
        self._h = h
        dims, rope = N.Dims(), N.GgufRope()
        if lib.camelid_gguf_model(h, max_pos, C.byref(dims), C.byref(rope)):
            msg = lib.camelid_gguf_last_error().decode()
            self.close()
            raise ValueError(msg)
        if dims.rope_dim != dims.head_dim:
            self.close()
            raise ValueError("partial RoPE (rope.dimension_count != head_dim) is not on the resident path")
        emb = self.tensor("token_embd.weight")
        out = self.tensor("output.weight") if self.has_tensor("output.weight") else emb
        kinds = {0: "none", 1: "linear", 2: "llama3"}
        self.cfg = ModelConfig(
            name=Path(str(path)).stem, n_layers=dims.n_layers, hidden=dims.hidden, ffn_dim=dims.ffn_dim,
            n_heads=dims.n_heads, n_kv_heads=dims.n_kv_heads, head_dim=dims.head_dim, vocab=dims.vocab,
            rope_theta=float(rope.freq_base), eps=float(dims.eps), tied=not self.has_tensor("output.weight"),
            qk_norm=self.has_tensor("blk.0.attn_q_norm.weight"), split_half=bool(dims.split_half_pairing),
            rope_scaling=kinds[rope.scaling_kind], rope_factor=float(rope.factor), rope_orig_ctx=float(rope.orig_ctx),
            rope_low=float(rope.low), rope_high=float(rope.high),
            # (the byte accounting of the benchmark; the engine takes each tensor's own format)
            quant_scheme="q8_0" if emb.type == 8 and out.type == 8 else "q4_k_m")
        self._embd = emb
        self._embd_quant = GGML_TO_QUANT.get(emb.type)
        self._freqs = None
        if rope.freqs:
            self._freqs = np.ctypeslib.as_array(C.cast(rope.freqs, C.POINTER(C.c_float)),
                                                (dims.rope_dim // 2,)).copy()

    def has_tensor(self, name: str) -> bool:
        t = N.GgufTensor()
        return self._lib.camelid_gguf_find(self._h, name.encode(), C.byref(t)) == 0

    def tensor(self, name: str) -> "N.GgufTensor":
        t = N.GgufTensor()
        if self._lib.camelid_gguf_find(self._h, name.encode(), C.byref(t)):
            raise KeyError(name)
        return t

    def tensor_bytes(self, name: str) -> np.ndarray:
        """A tensor's bytes as a read-only view of the mapping (valid until close)."""
        t = self.tensor(name)
        a = np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_uint8)), (t.n_bytes,))
        a.flags.writeable = False
        return a

    def rope_tables(self, pos0: int, n_pos: int):
        return rope_tables(self.cfg, pos0, n_pos, self._freqs)

    def embed(self, tokens) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty((len(toks), self.cfg.hidden), np.float32)
        data = C.cast(self._embd.data, C.POINTER(C.c_uint8))
        if self._embd_quant == Q8_0:
            rc = self._lib.camelid_embed_q8_0(data, self.cfg.vocab, self.cfg.hidden, N.ptr(toks, C.c_uint32),
                                              len(toks), N.ptr(out, C.c_float))
        elif self._embd_quant in (Q4_K, Q6_K):
            rc = self._lib.camelid_embed_kquant(self._embd_quant, data, self.cfg.vocab, self.cfg.hidden,
                                                N.ptr(toks, C.c_uint32), len(toks), N.ptr(out, C.c_float))
        else:
            raise ValueError(f"token_embd GGML type {self._embd.type} is not supported")
        if rc:
            raise ValueError("token id out of range")
        return out

    def load_into(self, eng: HipResidentDecode, device_embedding: bool = False) -> None:
        if self._lib.camelid_hip_load_gguf(eng._h, self._h, int(device_embedding)):
            raise N.HipError(self._lib.camelid_gguf_last_error().decode())

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.camelid_gguf_close(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


class ResidentSession:
    """Greedy generation over HipResidentDecode, mirroring the seam's loop (inference.rs:4383-4425)."""

    def __init__(self, model: SyntheticModel, max_pos: int | None = None, device_loop: bool = False):
        self.model = model
        self.cfg = model.cfg
        self.engine = HipResidentDecode(self.cfg.engine_dims(max_pos))
        model.load_into(self.engine, device_embedding=device_loop)
        self.device_loop = device_loop
        if device_loop:
            cos, sin = model.rope_tables(0, self.engine.max_pos())
            self.engine.set_rope_table(cos, sin)

    def prefill(self, tokens) -> None:
        n = len(tokens)
        if n == 0:
            return
        base = self.engine.filled()
        cos, sin = self.model.rope_tables(base, n)
        self.engine.prefill(self.model.embed(tokens), cos, sin, self.cfg.scale())

    def step(self, token: int, pos: int, logits: bool = False):
        cos, sin = self.model.rope_tables(pos, 1)
        emb = self.model.embed([token])[0]
        return self.engine.forward_token(emb, cos[0], sin[0], pos, self.cfg.scale(), compute_logits=logits)

    def generate(self, prompt, n_new: int) -> list[int]:
        prompt = [int(t) for t in prompt]
        self.engine.set_filled(0)
        self.prefill(prompt[:-1])
        pos = len(prompt) - 1
        if self.device_loop:
            return [int(t) for t in self.engine.generate(prompt[-1], pos, n_new, self.cfg.scale())]
        out = []
        tok = prompt[-1]
        for _ in range(n_new):
            tok = self.step(tok, pos)
            out.append(tok)
            pos += 1
        return out

    def close(self) -> None:
        self.engine.close()


def tiny_config(**kw) -> ModelConfig:
    """A small llama-shaped config for fast parity tests."""
    base = dict(name="tiny", n_layers=2, hidden=256, ffn_dim=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
                rope_theta=10000.0, seed=11, prompt_seed=12, prompt_len=16, decode_len=16)
    base.update(kw)
    return ModelConfig(**base)
