"""camelid_hip_attention_decode_split_noalloc (no reference counterpart: the split decode
attention for callers that cannot allocate) against camelid_hip_attention_decode_split, the
allocating entry point over the same kernels: bit-identical outputs on two calls in a row,
the second smaller than the first, so that nothing the first call left in the shared static
scratch can reach the second's result.  Both are also checked against the CPU oracle.
"""
import numpy as np
import pytest


def _dev(a):
    from camelid_amd.engine import DeviceBuffer
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _buf(nbytes):
    from camelid_amd.engine import DeviceBuffer
    return DeviceBuffer(nbytes)


def _ok(rc):
    from camelid_amd._native import check
    check(rc)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _case(orc, nh, nkv, hd, P, seed):
    rng = np.random.default_rng(seed)
    L, layer, max_pos = 2, 1, (P + 7) // 8 * 8
    kb = orc.f32_to_f16(rng.normal(0, 1.5, (L, nkv, max_pos, hd)).astype(np.float32))
    vb = orc.f32_to_f16(rng.normal(0, 1, (L, nkv, max_pos, hd)).astype(np.float32))
    q = rng.normal(0, 1, nh * hd).astype(np.float32)
    # device layout: K granules of 8 dims per position, V granules of 8 positions per dim
    kd = kb.reshape(L, nkv, max_pos, hd // 8, 8).transpose(0, 1, 3, 2, 4)
    vd = vb.reshape(L, nkv, max_pos // 8, 8, hd).transpose(0, 1, 2, 4, 3)
    want = orc.attention(q, orc.f16_to_f32(kb[layer]).ravel(), orc.f16_to_f32(vb[layer]).ravel(), nh, nkv, hd,
                         max_pos, P)
    return dict(nh=nh, nkv=nkv, hd=hd, P=P, layer=layer, max_pos=max_pos, q=_dev(q), k=_dev(kd), v=_dev(vd),
                pos=_dev(np.array([P - 1], np.uint32)), scale=float(np.float32(1) / np.sqrt(np.float32(hd))),
                want=want)


def _run(entry, c):
    nh, hd = c["nh"], c["hd"]
    out, xq, xs = _buf(nh * hd * 4), _buf(nh * hd), _buf(nh * hd // 32 * 4)
    _ok(entry(c["q"].ptr, c["k"].ptr, c["v"].ptr, c["layer"], nh, c["nkv"], hd, c["max_pos"], c["pos"].ptr,
              c["scale"], out.ptr, xq.ptr, xs.ptr, None))
    return (out.download(np.float32, nh * hd), xq.download(np.int8, nh * hd),
            xs.download(np.float32, nh * hd // 32))


@pytest.mark.gpu
def test_noalloc_split_attention_matches_allocating_entry(native, orc):
    # first call at the scratch limit (n_heads * max_pos = 2^20 score words), second smaller
    cases = [(64, 8, 64, 16384, 11), (24, 8, 128, 511, 12)]
    for nh, nkv, hd, P, seed in cases:
        print(f"[no_alloc] nh={nh} nkv={nkv} hd={hd} P={P}", flush=True)
        c = _case(orc, nh, nkv, hd, P, seed)
        got = _run(native.camelid_hip_attention_decode_split_noalloc, c)
        ref = _run(native.camelid_hip_attention_decode_split, c)
        assert np.array_equal(_bits(got[0]), _bits(ref[0]))
        assert np.array_equal(got[1], ref[1])
        assert np.array_equal(_bits(got[2]), _bits(ref[2]))
        assert np.array_equal(_bits(got[0]), _bits(c["want"]))


def test_noalloc_split_attention_refuses_oversize(native):
    """Runs without a GPU: the size check comes before any HIP call."""
    from camelid_amd._native import HipError
    # 64 heads x 16392 positions: one KV row past the 2^20-word score scratch, refused before any launch
    with pytest.raises(HipError, match="static scratch"):
        _ok(native.camelid_hip_attention_decode_split_noalloc(8, 8, 8, 0, 64, 8, 64, 16392, 8, 1.0, 8, 8, 8, None))
