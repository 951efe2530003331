"""akv_hip_decode_attention_noalloc (workspace in the library's static device
array) against akv_hip_decode_attention_fused (caller workspace), both
called through the C-ABI: identical outputs, bit for bit (same kernels and
schedule), over consecutive calls of different sizes (the array keeps the last
call's states; the arrival counters must come back to zero), plus the size
limits rejected before anything runs."""
import ctypes as ct

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from astc_kv.gpu import LIB_PATH, AkvAttnParams  # noqa: E402


def _noalloc(lib):
    fn = lib.akv_hip_decode_attention_noalloc
    fn.argtypes = [ct.POINTER(AkvAttnParams)] + [ct.c_void_p] * 7
    fn.restype = ct.c_int
    return fn


def _case(seed, b, hq, hkv, t, d, layout, block):
    from astc_kv import gpu
    from astc_kv.atlas import build_atlas
    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.normal(size=(b, hq, d)).astype(np.float32)).cuda()
    k = torch.from_numpy(rng.normal(size=(b, hkv, t, d)).astype(np.float16)).cuda()
    v = rng.normal(0, 0.5, size=(b, hkv, t, d)).astype(np.float32)
    atlas = gpu.DeviceAtlas.from_host(build_atlas(v, layout, block, page_tokens=120, quality=20))
    return q, k, atlas, gpu.make_params(atlas, hq)


@pytest.mark.gpu
def test_noalloc_matches_fused_entry_point():
    from astc_kv import gpu
    lib = gpu.lib()
    noalloc = _noalloc(lib)
    big = _case(1, 4, 9, 3, 3000, 64, "rgba", (6, 5))
    small = _case(2, 2, 8, 2, 777, 128, "scalar", (6, 6))
    for name, (q, k, atlas, params) in (("first", big), ("second, smaller", small), ("third, larger again", big)):
        print(f"no-alloc call: {name}: batch {params.batch} T{params.tokens} D{params.dim} {params.splits} splits",
              flush=True)
        want = gpu.decode_attention(q, k, atlas, params=params)             # akv_hip_decode_attention_fused
        got = torch.full_like(want, float("nan"))
        stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = noalloc(ct.byref(params), q.data_ptr(), k.data_ptr(), atlas.blocks.data_ptr(), atlas.scale.data_ptr(),
                     atlas.offset.data_ptr(), got.data_ptr(), stream)
        assert rc == 0, lib.akv_hip_error_string(rc)
        torch.cuda.synchronize()
        assert torch.equal(got, want), name


def test_noalloc_limits_rejected_before_any_launch():
    # Fake, aligned device addresses: the size checks return first, so this
    # runs without a GPU.
    lib = ct.CDLL(str(LIB_PATH))
    noalloc = _noalloc(lib)
    lib.akv_hip_error_string.argtypes = [ct.c_int]
    lib.akv_hip_error_string.restype = ct.c_char_p
    ptrs = [0x10000 * (i + 1) for i in range(6)] + [None]
    # T32768 x batch 64, 32q/8kv, D128, 2048-token splits: 64*32*16*130*4 B = 17 MB of states.
    p = AkvAttnParams(64, 32768, 32, 8, 128, 128, 2048, 16, 1, 4, 4, 8192, 8)
    assert noalloc(ct.byref(p), *ptrs) == -6
    assert b"static scratch" in lib.akv_hip_error_string(-6)
    # Invalid parameters keep their own codes.
    p = AkvAttnParams(1, 384, 9, 3, 96, 120, 48, 8, 1, 6, 5, 77, 3)
    assert noalloc(ct.byref(p), *ptrs) == -2
