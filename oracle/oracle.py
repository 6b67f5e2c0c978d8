"""ctypes wrapper of the CPU oracle (oracle/camelid_oracle.cpp).  TEST INFRASTRUCTURE ONLY.

Builds oracle/_build/libcamelid_oracle.so on first use when missing (g++ is present
wherever the tests run).  The product package never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libcamelid_oracle.so"
# tests/test_oracle_mutants.py points this at deliberately altered builds of the oracle
LIB_OVERRIDE = os.environ.get("CAMELID_ORACLE_LIB")

f32p = C.POINTER(C.c_float)
u8p = C.POINTER(C.c_uint8)
i8p = C.POINTER(C.c_int8)
u16p = C.POINTER(C.c_uint16)
u32p = C.POINTER(C.c_uint32)
i32p = C.POINTER(C.c_int32)
vp = C.c_void_p

_SIG = {
    "oracle_f32_to_f16": (C.c_uint16, [C.c_float]),
    "oracle_f16_to_f32": (C.c_float, [C.c_uint16]),
    "oracle_f32_to_f16_n": (None, [f32p, u16p, C.c_size_t]),
    "oracle_f16_to_f32_n": (None, [u16p, f32p, C.c_size_t]),
    "oracle_expf_n": (None, [f32p, f32p, C.c_size_t]),
    "oracle_quantize_q8_0": (None, [f32p, C.c_size_t, f32p, i8p]),
    "oracle_quantize_q8_0_wire": (None, [f32p, C.c_size_t, u8p]),
    "oracle_dequant_q8_0_wire": (None, [u8p, C.c_size_t, f32p]),
    "oracle_q8_block_dot": (C.c_int32, [i8p, i8p]),
    "oracle_q8_0_block_dots": (None, [u8p, C.c_size_t, C.c_size_t, i8p, i32p]),
    "oracle_q8_0_gemv": (None, [u8p, C.c_size_t, C.c_size_t, f32p, i8p, f32p]),
    "oracle_q8_0_gemm": (None, [u8p, C.c_size_t, C.c_size_t, C.c_size_t, f32p, i8p, f32p]),
    "oracle_rms_norm": (None, [f32p, f32p, C.c_size_t, C.c_size_t, C.c_float, f32p]),
    "oracle_rope_tables": (None, [C.c_uint32, C.c_float, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float, f32p,
                                  C.c_uint32, C.c_uint32, f32p, f32p]),
    "oracle_rope_frequencies": (None, [C.c_uint32, C.c_float, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float,
                                       f32p, f32p]),
    "oracle_apply_rope": (None, [f32p, C.c_uint32, C.c_uint32, C.c_uint32, f32p, f32p, C.c_int]),
    "oracle_silu_mul": (None, [f32p, f32p, C.c_size_t, f32p]),
    "oracle_argmax": (C.c_uint32, [f32p, C.c_size_t]),
    "oracle_attention": (None, [f32p, f32p, f32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, f32p]),
    "oracle_model_new": (vp, [C.c_uint32] * 8 + [C.c_float, C.c_int]),
    "oracle_model_free": (None, [vp]),
    "oracle_model_set_layer": (None, [vp, C.c_uint32] + [u8p] * 7 + [f32p] * 4),
    "oracle_model_set_output": (None, [vp, f32p, u8p, u8p]),
    "oracle_model_embed": (None, [vp, C.c_uint32, f32p]),
    "oracle_model_forward": (C.c_int, [vp, f32p, C.c_uint32, f32p, f32p, f32p, f32p, u32p]),
    "oracle_model_read_kv": (None, [vp, C.c_uint32, C.c_uint32, f32p, f32p]),
    "oracle_model_seed_kv": (None, [vp, C.c_uint32, C.c_uint32, f32p, f32p]),
    "oracle_serial_sum_rows": (None, [f32p, C.c_size_t, C.c_size_t, f32p]),
    "oracle_quantize_q8_k": (None, [f32p, C.c_size_t, f32p, i8p]),
    "oracle_nearest_int": (C.c_int32, [C.c_float]),
    "oracle_dequant_q4_k": (None, [u8p, C.c_size_t, f32p]),
    "oracle_dequant_q6_k": (None, [u8p, C.c_size_t, f32p]),
    "oracle_kquant_gemv": (None, [C.c_int, u8p, C.c_size_t, C.c_size_t, f32p, i8p, f32p]),
    "oracle_model_set_quant": (None, [vp, C.c_uint32, u8p]),
    "oracle_model_set_output_quant": (None, [vp, C.c_int, C.c_int]),
    "oracle_set_threads": (None, [C.c_int]),
}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if LIB_OVERRIDE:
            h = C.CDLL(LIB_OVERRIDE)
        else:
            if not LIB_PATH.exists():
                build()
            h = C.CDLL(str(LIB_PATH))
        for n, (r, a) in _SIG.items():
            fn = getattr(h, n)
            fn.restype = r
            fn.argtypes = a
        _lib = h
    return _lib


def set_threads(n: int) -> None:
    """OpenMP threads of the oracle's row-parallel loops (no effect on any result)."""
    lib().oracle_set_threads(int(n))


def P(a, t):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(t))


# ---------------------------------------------------------------- scalar / vector helpers
def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16_n(P(x, C.c_float), P(out, C.c_uint16), x.size)
    return out


def f16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_f16_to_f32_n(P(b, C.c_uint16), P(out, C.c_float), b.size)
    return out


def expf(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().oracle_expf_n(P(x, C.c_float), P(out, C.c_float), x.size)
    return out


def quantize_q8_0(x):
    """-> (scales f32 [n/32], quants i8 [n])."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    s = np.empty(x.size // 32, np.float32)
    q = np.empty(x.size, np.int8)
    lib().oracle_quantize_q8_0(P(x, C.c_float), x.size, P(s, C.c_float), P(q, C.c_int8))
    return s, q


def quantize_q8_0_wire(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().oracle_quantize_q8_0_wire(P(x, C.c_float), x.size, P(out, C.c_uint8))
    return out


def dequant_q8_0_wire(wire) -> np.ndarray:
    wire = np.ascontiguousarray(wire, np.uint8)
    nb = wire.size // 34
    out = np.empty(nb * 32, np.float32)
    lib().oracle_dequant_q8_0_wire(P(wire, C.c_uint8), nb, P(out, C.c_float))
    return out


def q8_0_block_dots(wire, rows, k, xq) -> np.ndarray:
    out = np.empty((rows, k // 32), np.int32)
    lib().oracle_q8_0_block_dots(P(np.ascontiguousarray(wire, np.uint8), C.c_uint8), rows, k,
                                 P(np.ascontiguousarray(xq, np.int8), C.c_int8), P(out, C.c_int32))
    return out


def q8_0_gemv(wire, rows, k, xs, xq) -> np.ndarray:
    out = np.empty(rows, np.float32)
    lib().oracle_q8_0_gemv(P(np.ascontiguousarray(wire, np.uint8), C.c_uint8), rows, k,
                           P(np.ascontiguousarray(xs, np.float32), C.c_float),
                           P(np.ascontiguousarray(xq, np.int8), C.c_int8), P(out, C.c_float))
    return out


def q8_0_gemm(wire, rows, k, xs, xq) -> np.ndarray:
    """xs [T][k/32], xq [T][k] -> [T][rows]."""
    xs = np.ascontiguousarray(xs, np.float32)
    xq = np.ascontiguousarray(xq, np.int8)
    T = xs.shape[0]
    out = np.empty((T, rows), np.float32)
    lib().oracle_q8_0_gemm(P(np.ascontiguousarray(wire, np.uint8), C.c_uint8), rows, k, T, P(xs, C.c_float),
                           P(xq, C.c_int8), P(out, C.c_float))
    return out


def quantize_q8_k(x):
    """-> (scales f32 [n/256], quants i8 [n]) (inference.rs:17564-17599)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    d = np.empty(x.size // 256, np.float32)
    q = np.empty(x.size, np.int8)
    lib().oracle_quantize_q8_k(P(x, C.c_float), x.size, P(d, C.c_float), P(q, C.c_int8))
    return d, q


def nearest_int(x: float) -> int:
    return int(lib().oracle_nearest_int(float(x)))


def dequant_kquant(quant: int, wire) -> np.ndarray:
    wire = np.ascontiguousarray(wire, np.uint8)
    nsb = wire.size // (144 if quant == 1 else 210)
    out = np.empty(nsb * 256, np.float32)
    fn = lib().oracle_dequant_q4_k if quant == 1 else lib().oracle_dequant_q6_k
    fn(P(wire, C.c_uint8), nsb, P(out, C.c_float))
    return out


def kquant_gemv(quant: int, wire, rows, k, yd, yq) -> np.ndarray:
    out = np.empty(rows, np.float32)
    lib().oracle_kquant_gemv(quant, P(np.ascontiguousarray(wire, np.uint8), C.c_uint8), rows, k,
                             P(np.ascontiguousarray(yd, np.float32), C.c_float),
                             P(np.ascontiguousarray(yq, np.int8), C.c_int8), P(out, C.c_float))
    return out


def serial_sum_rows(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    out = np.empty(rows, np.float32)
    lib().oracle_serial_sum_rows(P(x, C.c_float), rows, n, P(out, C.c_float))
    return out


def rms_norm(x, w, eps) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    rows = 1 if x.ndim == 1 else x.shape[0]
    out = np.empty_like(x)
    lib().oracle_rms_norm(P(x, C.c_float), P(w, C.c_float), rows, x.shape[-1], eps, P(out, C.c_float))
    return out


def rope_tables(rope_dim, base, kind=0, factor=1.0, orig_ctx=8192.0, low=1.0, high=4.0, freqs=None, pos0=0, n_pos=1):
    half = rope_dim // 2
    c = np.empty((n_pos, half), np.float32)
    s = np.empty((n_pos, half), np.float32)
    fp = P(np.ascontiguousarray(freqs, np.float32), C.c_float) if freqs is not None else None
    lib().oracle_rope_tables(rope_dim, base, kind, factor, orig_ctx, low, high, fp, pos0, n_pos, P(c, C.c_float),
                             P(s, C.c_float))
    return c, s


def rope_frequencies(rope_dim, base, kind=0, factor=1.0, orig_ctx=8192.0, low=1.0, high=4.0, freqs=None):
    """The per-pair frequencies theta_i that rope_tables() takes cos/sin of."""
    out = np.empty(rope_dim // 2, np.float32)
    fp = P(np.ascontiguousarray(freqs, np.float32), C.c_float) if freqs is not None else None
    lib().oracle_rope_frequencies(rope_dim, base, kind, factor, orig_ctx, low, high, fp, P(out, C.c_float))
    return out


def apply_rope(x, heads, hd, rope_dim, cos, sin, split_half=False) -> np.ndarray:
    out = np.array(x, np.float32, copy=True).ravel()
    lib().oracle_apply_rope(P(out, C.c_float), heads, hd, rope_dim, P(np.ascontiguousarray(cos, np.float32), C.c_float),
                            P(np.ascontiguousarray(sin, np.float32), C.c_float), int(split_half))
    return out


def silu_mul(g, u) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().oracle_silu_mul(P(g, C.c_float), P(u, C.c_float), g.size, P(out, C.c_float))
    return out


def argmax(x) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().oracle_argmax(P(x, C.c_float), x.size))


def attention(q, kc, vc, n_heads, n_kv, hd, max_pos, n_pos) -> np.ndarray:
    out = np.empty(n_heads * hd, np.float32)
    lib().oracle_attention(P(np.ascontiguousarray(q, np.float32), C.c_float),
                           P(np.ascontiguousarray(kc, np.float32), C.c_float),
                           P(np.ascontiguousarray(vc, np.float32), C.c_float), n_heads, n_kv, hd, max_pos, n_pos,
                           P(out, C.c_float))
    return out


# ---------------------------------------------------------------- model
class OracleModel:
    """CPU forward over a SyntheticModel's weights (Q8_0 wire bytes; borrowed, kept alive here)."""

    def __init__(self, model, max_pos: int):
        cfg = model.cfg
        self.cfg = cfg
        self.model = model
        self.max_pos = max_pos
        L = lib()
        self.h = L.oracle_model_new(cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.hidden, cfg.ffn_dim,
                                    cfg.vocab, max_pos, cfg.eps, int(cfg.split_half))
        self._keep = []
        for i, layer in enumerate(model.layers):
            pj = layer["projs"]
            ws = [P(pj[n], C.c_uint8) for n in ("q", "k", "v", "o", "gate", "up", "down")]
            norms = [layer["attn_norm"], layer["ffn_norm"], layer.get("q_norm"), layer.get("k_norm")]
            nptr = [P(a, C.c_float) if a is not None else None for a in norms]
            L.oracle_model_set_layer(self.h, i, *ws, *nptr)
            q7 = np.ascontiguousarray(layer.get("quant", [0] * 7), np.uint8)
            self._keep.append(q7)
            L.oracle_model_set_quant(self.h, i, P(q7, C.c_uint8))
        L.oracle_model_set_output(self.h, P(model.output_norm, C.c_float), P(model.output, C.c_uint8),
                                  P(model.token_embd, C.c_uint8))
        L.oracle_model_set_output_quant(self.h, cfg.output_quant(), cfg.embd_quant())
        kind = {"none": 0, "linear": 1, "llama3": 2}[cfg.rope_scaling]
        self.cos, self.sin = rope_tables(cfg.rope_dim, cfg.rope_theta, kind, cfg.rope_factor, cfg.rope_orig_ctx,
                                         cfg.rope_low, cfg.rope_high, None, 0, max_pos)

    def close(self):
        if self.h:
            lib().oracle_model_free(self.h)
            self.h = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def embed(self, tok: int) -> np.ndarray:
        out = np.empty(self.cfg.hidden, np.float32)
        lib().oracle_model_embed(self.h, tok, P(out, C.c_float))
        return out

    def forward(self, tok: int, pos: int, hidden=False, logits=False):
        """One step; returns (token, hidden [L+1][H] or None, logits [V] or None)."""
        cfg = self.cfg
        emb = self.embed(tok)
        hid = np.empty((cfg.n_layers + 1, cfg.hidden), np.float32) if hidden else None
        lg = np.empty(cfg.vocab, np.float32) if logits else None
        t = C.c_uint32(0)
        rc = lib().oracle_model_forward(self.h, P(emb, C.c_float), pos, P(np.ascontiguousarray(self.cos[pos]), C.c_float),
                                        P(np.ascontiguousarray(self.sin[pos]), C.c_float),
                                        P(hid, C.c_float) if hid is not None else None,
                                        P(lg, C.c_float) if lg is not None else None, C.byref(t))
        if rc:
            raise ValueError("position out of range")
        return int(t.value), hid, lg

    def prefill(self, tokens, pos0: int = 0) -> None:
        L = lib()
        for i, tok in enumerate(tokens):
            emb = self.embed(int(tok))
            p = pos0 + i
            L.oracle_model_forward(self.h, P(emb, C.c_float), p, P(np.ascontiguousarray(self.cos[p]), C.c_float),
                                   P(np.ascontiguousarray(self.sin[p]), C.c_float), None, None, None)

    def generate(self, prompt, n_new: int, margins: list | None = None) -> list[int]:
        """Prefill n-1 prompt tokens, then n_new greedy steps (inference.rs:4383-4425)."""
        prompt = [int(t) for t in prompt]
        self.prefill(prompt[:-1])
        pos = len(prompt) - 1
        tok = prompt[-1]
        out = []
        for _ in range(n_new):
            want = margins is not None
            tok, _, lg = self.forward(tok, pos, logits=want)
            if want:
                top2 = np.partition(lg, -2)[-2:]
                margins.append(float(top2[1] - top2[0]))
            out.append(tok)
            pos += 1
        return out

    def read_kv(self, layer: int, n: int):
        cfg = self.cfg
        k = np.empty((cfg.n_kv_heads, n, cfg.head_dim), np.float32)
        v = np.empty_like(k)
        lib().oracle_model_read_kv(self.h, layer, n, P(k, C.c_float), P(v, C.c_float))
        return k, v

    def seed_kv(self, layer: int, k, v) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        lib().oracle_model_seed_kv(self.h, layer, k.shape[1], P(k, C.c_float), P(v, C.c_float))
