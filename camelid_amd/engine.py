"""HipResidentDecode: Python mirror of Camelid's `CudaResidentDecode` over the C ABI.

Method names, argument meaning and error behaviour follow src/cuda_resident.rs:
every method raises HipError where the reference returns Err(String), which the seam
turns into "decline -> CPU fallback" (inference.rs:3316-3371).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _native as N

PROJ_NAMES = ("q", "k", "v", "o", "gate", "up", "down")
Q8_0, Q4_K, Q6_K = 0, 1, 2
WIRE34, BLOCK36 = 34, 36


@dataclass(frozen=True)
class EngineDims:
    """Arguments of CudaResidentDecode::new (cuda_resident.rs:5601)."""

    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    hidden: int
    ffn_dim: int
    rope_dim: int
    max_pos: int
    vocab: int
    eps: float
    split_half_pairing: bool = False

    def to_c(self) -> N.Dims:
        return N.Dims(self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim, self.hidden, self.ffn_dim,
                      self.rope_dim, self.max_pos, self.vocab, self.eps, int(self.split_half_pairing))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


def _sized(a: np.ndarray, count: int, what: str) -> np.ndarray:
    """a, refused unless it holds exactly `count` values: the C side copies fixed sizes
    derived from the model dims (the reference's prefill checks these lengths,
    cuda_resident.rs:7795)."""
    if a.size != count:
        raise ValueError(f"{what}: {a.size} values, expected {count}")
    return a


def _rows(a: np.ndarray, width: int, what: str) -> int:
    """Number of rows of width `width` in a (a 1-D array is one row); refuses other shapes."""
    if a.ndim == 1:
        a = a.reshape(1, -1)
    if a.ndim != 2 or a.shape[1] != width:
        raise ValueError(f"{what}: shape {a.shape}, expected [n][{width}]")
    return a.shape[0]


class HipResidentDecode:
    """Resident weights + f16 KV cache on one MI355X; one stream, one sync per call."""

    def __init__(self, dims: EngineDims):
        self.dims = dims
        self._lib = N.lib()
        h = N.vp()
        cd = dims.to_c()
        N.check(self._lib.camelid_hip_engine_new(C.byref(cd), C.byref(h)))
        self._h = h

    # -- lifecycle ---------------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.camelid_hip_engine_free(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _chk(self, rc: int) -> None:
        N.check(rc, self._h)

    # -- weights (cuda_resident.rs:5801 set_layer_located, :6008 set_output) ---------------
    def set_layer(self, layer: int, projs: dict, attn_norm, ffn_norm, q_norm=None, k_norm=None,
                  q8_layout: int = WIRE34, quants=None) -> None:
        arrs = [_u8(projs[n]) for n in PROJ_NAMES]
        ptrs = (N.u8p * 7)(*[N.ptr(a, C.c_uint8) for a in arrs])
        lens = (C.c_size_t * 7)(*[a.nbytes for a in arrs])
        qs = (C.c_uint8 * 7)(*(quants or [Q8_0] * 7))
        d = self.dims
        an = _sized(_f32(attn_norm), d.hidden, "attn_norm")
        fn = _sized(_f32(ffn_norm), d.hidden, "ffn_norm")
        qn = _sized(_f32(q_norm), d.head_dim, "q_norm") if q_norm is not None else None
        kn = _sized(_f32(k_norm), d.head_dim, "k_norm") if k_norm is not None else None
        self._chk(self._lib.camelid_hip_set_layer(
            self._h, layer, ptrs, lens, qs, q8_layout, N.ptr(an, C.c_float), N.ptr(fn, C.c_float),
            N.ptr(qn, C.c_float) if qn is not None else None, N.ptr(kn, C.c_float) if kn is not None else None))

    def set_output(self, final_norm, weight, quant: int = Q8_0, q8_layout: int = WIRE34) -> None:
        fn, w = _sized(_f32(final_norm), self.dims.hidden, "final_norm"), _u8(weight)
        self._chk(self._lib.camelid_hip_set_output(self._h, N.ptr(fn, C.c_float), N.ptr(w, C.c_uint8), w.nbytes,
                                                   quant, q8_layout))

    def set_embedding(self, weight, quant: int = Q8_0, q8_layout: int = WIRE34) -> None:
        w = _u8(weight)
        self._chk(self._lib.camelid_hip_set_embedding(self._h, N.ptr(w, C.c_uint8), w.nbytes, quant, q8_layout))

    def set_rope_table(self, cos_all, sin_all) -> None:
        c, s = _f32(cos_all), _f32(sin_all)
        half = self.dims.rope_dim // 2
        n = _rows(c, half, "cos_all")
        if _rows(s, half, "sin_all") != n:
            raise ValueError("cos_all and sin_all must have the same number of rows")
        self._chk(self._lib.camelid_hip_set_rope_table(self._h, N.ptr(c, C.c_float), N.ptr(s, C.c_float), n))

    # -- state (cuda_resident.rs:6261-6292) ------------------------------------------------
    def weights_ready(self) -> bool:
        return bool(self._lib.camelid_hip_weights_ready(self._h))

    def filled(self) -> int:
        return int(self._lib.camelid_hip_filled(self._h))

    def set_filled(self, n: int) -> None:
        self._chk(self._lib.camelid_hip_set_filled(self._h, n))

    def max_pos(self) -> int:
        return int(self._lib.camelid_hip_max_pos(self._h))

    def n_layers(self) -> int:
        return int(self._lib.camelid_hip_n_layers(self._h))

    def uses_kquant(self) -> bool:
        return bool(self._lib.camelid_hip_uses_kquant(self._h))

    # -- KV handoff (cuda_resident.rs:6305 seed_layer, :6348 read_kv_layer) ----------------
    def seed_layer(self, layer: int, ck, cv, n_pos: int) -> None:
        d = self.dims
        k = _sized(_f32(ck), d.n_kv_heads * n_pos * d.head_dim, "ck")
        v = _sized(_f32(cv), d.n_kv_heads * n_pos * d.head_dim, "cv")
        self._chk(self._lib.camelid_hip_seed_layer(self._h, layer, N.ptr(k, C.c_float), N.ptr(v, C.c_float), n_pos))

    def read_kv_layer(self, layer: int, n: int):
        d = self.dims
        k = np.empty((d.n_kv_heads, n, d.head_dim), np.float32)
        v = np.empty_like(k)
        self._chk(self._lib.camelid_hip_read_kv_layer(self._h, layer, n, N.ptr(k, C.c_float), N.ptr(v, C.c_float)))
        return k, v

    # -- forward (cuda_resident.rs:7430 forward_token, :7724 forward_token_logits) ---------
    def forward_token(self, embedding, cos, sin, position: int, scale: float, compute_logits: bool = True):
        """Returns the greedy token (and fills self.last_logits when compute_logits)."""
        d = self.dims
        e = _sized(_f32(embedding), d.hidden, "embedding")
        c = _sized(_f32(cos), d.rope_dim // 2, "cos")
        s = _sized(_f32(sin), d.rope_dim // 2, "sin")
        tok = C.c_uint32(0)
        logits = np.empty(self.dims.vocab, np.float32) if compute_logits else None
        self._chk(self._lib.camelid_hip_forward_token(
            self._h, N.ptr(e, C.c_float), N.ptr(c, C.c_float), N.ptr(s, C.c_float), position, scale,
            1 if compute_logits else 0, C.byref(tok), N.ptr(logits, C.c_float) if logits is not None else None))
        self.last_logits = logits
        return int(tok.value)

    def forward_token_logits(self, embedding, cos, sin, position: int, scale: float) -> np.ndarray:
        self.forward_token(embedding, cos, sin, position, scale, compute_logits=True)
        return self.last_logits

    def prefill(self, embeddings, cos_all, sin_all, scale: float) -> None:
        """Positions [filled, filled+n) (cuda_resident.rs:7785 prefill / :8797 prefill_batched)."""
        n = self._rows_checked(embeddings, cos_all, sin_all)
        e, c, s = _f32(embeddings), _f32(cos_all), _f32(sin_all)
        self._chk(self._lib.camelid_hip_prefill(self._h, N.ptr(e, C.c_float), N.ptr(c, C.c_float),
                                                N.ptr(s, C.c_float), n, scale))

    prefill_batched = prefill

    def _rows_checked(self, embeddings, cos_all, sin_all) -> int:
        """Rows of the [n][H] embeddings, refused unless cos/sin hold [n][rope_dim/2]."""
        d = self.dims
        n = _rows(np.asarray(embeddings), d.hidden, "embeddings")
        half = d.rope_dim // 2
        if _rows(np.asarray(cos_all), half, "cos_all") != n or _rows(np.asarray(sin_all), half, "sin_all") != n:
            raise ValueError(f"cos_all / sin_all must hold {n} rows of {half}")
        return n

    MAX_VERIFY_K = 8

    def verify_batch(self, embeddings, cos_all, sin_all, base_position: int, scale: float) -> np.ndarray:
        """k tokens at [base_position, base_position + k) in one batched forward; the greedy
        token after each (cuda_resident.rs:7821).  filled is left to the caller."""
        k = self._rows_checked(embeddings, cos_all, sin_all)
        e, c, s = _f32(embeddings), _f32(cos_all), _f32(sin_all)
        out = np.empty(k, np.uint32)
        self._chk(self._lib.camelid_hip_verify(self._h, N.ptr(e, C.c_float), N.ptr(c, C.c_float), N.ptr(s, C.c_float),
                                               base_position, k, scale, N.ptr(out, C.c_uint32)))
        return out

    def generate(self, token: int, position: int, n_steps: int, scale: float) -> np.ndarray:
        """Device-side greedy loop (forward_token_device, cuda_resident.rs:7529)."""
        out = np.empty(n_steps, np.uint32)
        self._chk(self._lib.camelid_hip_generate(self._h, token, position, n_steps, scale, N.ptr(out, C.c_uint32)))
        return out

    # -- measurement ------------------------------------------------------------------------
    # prefill_gemm: the prefill projections; its "bytes" are int8 operations
    PROFILE_CATEGORIES = ("gemv", "rmsnorm_quant", "attention", "silu_quant", "head", "embed", "prefill_gemm")

    def profile_begin(self) -> None:
        self._chk(self._lib.camelid_hip_profile_begin(self._h))

    def profile_end(self) -> dict:
        n = len(self.PROFILE_CATEGORIES)
        ms = (C.c_double * n)()
        by = (C.c_double * n)()
        ln = (C.c_uint64 * n)()
        self._chk(self._lib.camelid_hip_profile_end(self._h, ms, by, ln, n))
        return {c: {"ms": ms[i], "bytes": by[i], "launches": int(ln[i])}
                for i, c in enumerate(self.PROFILE_CATEGORIES)}

    # -- test hooks --------------------------------------------------------------------------
    def capture_hidden(self, enable: bool = True) -> None:
        self._chk(self._lib.camelid_hip_capture_hidden(self._h, 1 if enable else 0))

    def read_hidden(self) -> np.ndarray:
        d = self.dims
        out = np.empty((d.n_layers + 1, d.hidden), np.float32)
        self._chk(self._lib.camelid_hip_read_hidden(self._h, N.ptr(out, C.c_float)))
        return out


class DeviceBuffer:
    """A device allocation owned by Python (for kernel-level calls through the C ABI)."""

    def __init__(self, nbytes: int):
        self._lib = N.lib()
        p = N.vp()
        N.check(self._lib.camelid_hip_malloc(C.byref(p), max(int(nbytes), 1)))
        self.ptr = p
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than the buffer")
        N.check(self._lib.camelid_hip_memcpy_htod(self.ptr, a.ctypes.data_as(N.vp), a.nbytes))

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("read beyond the buffer")
        N.check(self._lib.camelid_hip_synchronize())
        N.check(self._lib.camelid_hip_memcpy_dtoh(out.ctypes.data_as(N.vp), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            self._lib.camelid_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):  # pragma: no cover
        try:
            self.free()
        except Exception:
            pass


def device_info() -> tuple[str, int]:
    buf = C.create_string_buffer(256)
    cu = C.c_int(0)
    N.check(N.lib().camelid_hip_device_info(buf, 256, C.byref(cu)))
    return buf.value.decode(), int(cu.value)
