"""ctypes bindings of the native library (include/camelid_hip.h).

The library is built in-tree by camelid_amd/build.py.  Loading fails loudly when it is
missing: there is no CPU fallback on the product path.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "_lib"
# The product library; CAMELID_HIP_LIB names another build of it in the same directory (the
# measurement build libcamelid_hip_stamps.so, which also records phase timestamps).
LIB_PATH = LIB_DIR / os.environ.get("CAMELID_HIP_LIB", "libcamelid_hip.so")

u8p = C.POINTER(C.c_uint8)
i8p = C.POINTER(C.c_int8)
u16p = C.POINTER(C.c_uint16)
u32p = C.POINTER(C.c_uint32)
f32p = C.POINTER(C.c_float)
vp = C.c_void_p


class Dims(C.Structure):
    """camelid_hip_dims: the arguments of CudaResidentDecode::new (cuda_resident.rs:5601)."""

    _fields_ = [
        ("n_layers", C.c_uint32),
        ("n_heads", C.c_uint32),
        ("n_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("hidden", C.c_uint32),
        ("ffn_dim", C.c_uint32),
        ("rope_dim", C.c_uint32),
        ("max_pos", C.c_uint32),
        ("vocab", C.c_uint32),
        ("eps", C.c_float),
        ("split_half_pairing", C.c_uint32),
    ]


class GgufTensor(C.Structure):
    """camelid_gguf_tensor: one entry of a mapped GGUF file's tensor directory."""

    _fields_ = [
        ("data", vp),
        ("n_bytes", C.c_uint64),
        ("offset", C.c_uint64),
        ("dims", C.c_uint64 * 4),
        ("n_dims", C.c_uint32),
        ("type", C.c_int32),
    ]


class GgufRope(C.Structure):
    """camelid_gguf_rope: a model's RoPE parameters in camelid_rope_tables' argument form."""

    _fields_ = [
        ("freq_base", C.c_float),
        ("scaling_kind", C.c_int32),
        ("factor", C.c_float),
        ("orig_ctx", C.c_float),
        ("low", C.c_float),
        ("high", C.c_float),
        ("freqs", vp),
    ]


# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    "camelid_hip_engine_new": (C.c_int, [C.POINTER(Dims), C.POINTER(vp)]),
    "camelid_hip_engine_free": (None, [vp]),
    "camelid_hip_check_model": (C.c_int, [C.POINTER(Dims), u8p, C.c_uint8]),
    "camelid_hip_last_error": (C.c_char_p, [vp]),
    "camelid_hip_set_layer": (C.c_int, [vp, C.c_uint32, C.POINTER(u8p), C.POINTER(C.c_size_t), u8p, C.c_uint8,
                                        f32p, f32p, f32p, f32p]),
    "camelid_hip_set_output": (C.c_int, [vp, f32p, u8p, C.c_size_t, C.c_uint8, C.c_uint8]),
    "camelid_hip_weights_ready": (C.c_int, [vp]),
    "camelid_hip_filled": (C.c_uint32, [vp]),
    "camelid_hip_set_filled": (C.c_int, [vp, C.c_uint32]),
    "camelid_hip_max_pos": (C.c_uint32, [vp]),
    "camelid_hip_n_layers": (C.c_uint32, [vp]),
    "camelid_hip_uses_kquant": (C.c_int, [vp]),
    "camelid_hip_seed_layer": (C.c_int, [vp, C.c_uint32, f32p, f32p, C.c_uint32]),
    "camelid_hip_read_kv_layer": (C.c_int, [vp, C.c_uint32, C.c_uint32, f32p, f32p]),
    "camelid_hip_forward_token": (C.c_int, [vp, f32p, f32p, f32p, C.c_uint32, C.c_float, C.c_int, u32p, f32p]),
    "camelid_hip_prefill": (C.c_int, [vp, f32p, f32p, f32p, C.c_uint32, C.c_float]),
    "camelid_hip_set_embedding": (C.c_int, [vp, u8p, C.c_size_t, C.c_uint8, C.c_uint8]),
    "camelid_hip_set_rope_table": (C.c_int, [vp, f32p, f32p, C.c_uint32]),
    "camelid_hip_generate": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, u32p]),
    "camelid_hip_capture_hidden": (C.c_int, [vp, C.c_int]),
    "camelid_hip_read_hidden": (C.c_int, [vp, f32p]),
    "camelid_hip_hbm_bandwidth": (C.c_int, [C.c_size_t, C.c_uint32, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "camelid_hip_profile_begin": (C.c_int, [vp]),
    "camelid_hip_profile_end": (C.c_int, [vp, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                          C.POINTER(C.c_uint64), C.c_uint32]),
    "camelid_hip_device_info": (C.c_int, [C.c_char_p, C.c_size_t, C.POINTER(C.c_int)]),
    "camelid_hip_phase_stamps": (C.c_int, [C.POINTER(C.c_uint64), C.c_size_t, C.POINTER(C.c_size_t)]),
    "camelid_hip_malloc": (C.c_int, [C.POINTER(vp), C.c_size_t]),
    "camelid_hip_free": (C.c_int, [vp]),
    "camelid_hip_memcpy_htod": (C.c_int, [vp, vp, C.c_size_t]),
    "camelid_hip_memcpy_dtoh": (C.c_int, [vp, vp, C.c_size_t]),
    "camelid_hip_synchronize": (C.c_int, []),
    "camelid_q8_0_repack": (C.c_int, [u8p, C.c_size_t, C.c_size_t, C.c_uint8, i8p, u16p]),
    "camelid_hip_q8_0_gemv": (C.c_int, [vp, vp, C.c_uint32, C.c_uint32, vp, vp, vp, vp, vp]),
    "camelid_hip_q8_0_block_dots": (C.c_int, [vp, C.c_uint32, C.c_uint32, vp, vp, vp]),
    "camelid_hip_rmsnorm_quantize": (C.c_int, [vp, vp, C.c_uint32, C.c_float, vp, vp, vp, vp]),
    "camelid_hip_quantize_q8_0": (C.c_int, [vp, C.c_uint32, vp, vp, vp]),
    "camelid_hip_silu_mul_quantize": (C.c_int, [vp, C.c_uint32, vp, vp, vp, vp]),
    "camelid_hip_rope_kv": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, vp,
                                      vp, C.c_float, vp, vp, vp, C.c_uint32, C.c_uint32, vp, vp]),
    "camelid_hip_attention_decode": (C.c_int, [vp, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                               C.c_uint32, vp, C.c_float, vp, vp, vp, vp]),
    "camelid_hip_attention_decode_split": (C.c_int, [vp, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                               C.c_uint32, vp, C.c_float, vp, vp, vp, vp]),
    "camelid_hip_attention_decode_split_noalloc": (C.c_int, [vp, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32,
                                                             C.c_uint32, C.c_uint32, vp, C.c_float, vp, vp, vp, vp]),
    "camelid_hip_q8_0_gemm": (C.c_int, [vp, vp, C.c_uint32, C.c_uint32, vp, vp, C.c_uint32, vp, vp, vp]),
    "camelid_hip_attention_prefill": (C.c_int, [vp, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                                C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, vp, vp, vp, vp]),
    "camelid_hip_quantize_q8_k": (C.c_int, [vp, C.c_uint32, vp, vp, vp, vp]),
    "camelid_hip_rmsnorm_q8_k": (C.c_int, [vp, vp, C.c_uint32, C.c_float, vp, vp, vp, vp]),
    "camelid_hip_silu_mul_q8_k": (C.c_int, [vp, C.c_uint32, vp, vp, vp, vp]),
    "camelid_kquant_repack": (C.c_int, [C.c_uint8, u8p, C.c_size_t, C.c_size_t, u8p, u8p, i8p, u16p]),
    "camelid_hip_kquant_gemv": (C.c_int, [C.c_uint8, vp, vp, vp, vp, C.c_uint32, C.c_uint32, vp, vp, vp, vp, vp,
                                          vp]),
    "camelid_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(vp)]),
    "camelid_gguf_close": (None, [vp]),
    "camelid_gguf_last_error": (C.c_char_p, []),
    "camelid_gguf_version": (C.c_uint32, [vp]),
    "camelid_gguf_alignment": (C.c_uint64, [vp]),
    "camelid_gguf_tensor_count": (C.c_uint64, [vp]),
    "camelid_gguf_tensor_name": (C.c_char_p, [vp, C.c_uint64]),
    "camelid_gguf_find": (C.c_int, [vp, C.c_char_p, C.POINTER(GgufTensor)]),
    "camelid_gguf_meta_u32": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_uint32)]),
    "camelid_gguf_meta_f32": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_float)]),
    "camelid_gguf_meta_str": (C.c_char_p, [vp, C.c_char_p]),
    "camelid_gguf_model": (C.c_int, [vp, C.c_uint32, C.POINTER(Dims), C.POINTER(GgufRope)]),
    "camelid_hip_load_gguf": (C.c_int, [vp, vp, C.c_int]),
    "camelid_hip_kquant_gemm": (C.c_int, [C.c_uint8, vp, vp, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp,
                                          vp, C.c_uint32, vp, vp]),
    "camelid_hip_time_kquant": (C.c_int, [C.c_uint8, vp, vp, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp,
                                          vp, C.c_uint32, C.POINTER(C.c_float)]),
    "camelid_hip_time_q8_0": (C.c_int, [C.c_int, C.POINTER(vp), C.POINTER(vp), C.c_uint32, C.c_uint32,
                                        C.c_uint32, vp, vp, C.c_uint32, vp, C.c_uint32, C.POINTER(C.c_float)]),
    "camelid_hip_argmax": (C.c_int, [vp, C.c_uint32, vp, vp]),
    "camelid_hip_rmsnorm_q8_0_gemv": (C.c_int, [vp, vp, C.c_uint32, C.c_uint32, vp, vp, C.c_float, vp, vp]),
    "camelid_hip_gate_up_silu": (C.c_int, [vp, vp, C.c_uint32, C.c_uint32, vp, vp, vp, vp, C.c_float, vp, vp, vp]),
    "camelid_hip_verify": (C.c_int, [vp, vp, vp, vp, C.c_uint32, C.c_uint32, C.c_float, vp]),
    "camelid_hip_inorder_sum_rows": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp]),
    "camelid_hip_expf": (C.c_int, [vp, vp, C.c_size_t, vp]),
    "camelid_expf_host": (None, [f32p, f32p, C.c_size_t]),
    # host seam + synthetic weights
    "camelid_rope_tables": (C.c_int, [C.c_uint32, C.c_float, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float,
                                      f32p, C.c_uint32, C.c_uint32, f32p, f32p]),
    "camelid_embed_q8_0": (C.c_int, [u8p, C.c_uint32, C.c_uint32, u32p, C.c_uint32, f32p]),
    "camelid_synth_normal_f32": (None, [C.c_char_p, C.c_uint64, C.c_float, f32p, C.c_uint64]),
    "camelid_synth_q8_0_wire": (C.c_int, [C.c_char_p, C.c_uint64, C.c_float, C.c_uint64, u8p]),
    "camelid_synth_tokens": (None, [C.c_uint64, C.c_uint32, C.c_uint32, u32p]),
    "camelid_synth_kquant_wire": (C.c_int, [C.c_char_p, C.c_uint64, C.c_float, C.c_uint64, C.c_int, u8p]),
    "camelid_embed_kquant": (C.c_int, [C.c_int, u8p, C.c_uint32, C.c_uint32, u32p, C.c_uint32, f32p]),
}

_lib = None


def lib() -> C.CDLL:
    """Load (once) and return the native library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python camelid_amd/build.py` "
                "(the HIP backend has no CPU fallback)")
        h = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def last_error(engine=None) -> str:
    msg = lib().camelid_hip_last_error(engine)
    return msg.decode() if msg else ""


class HipError(RuntimeError):
    pass


def check(rc: int, engine=None) -> None:
    if rc != 0:
        raise HipError(last_error(engine) or f"native call failed ({rc})")


def ptr(a, ctype):
    """ctypes pointer to a C-contiguous numpy array's data."""
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data_as(C.POINTER(ctype))
