"""The benchmark workloads at their configured sizes, with the default
schedules the host picks for them, on the GPU:

* T32768 x batch 8, 32 query / 8 KV heads, head dim 128, RGBA 4x4 V,
  Student-t (3 dof) K (default tile: 2048-token splits in two rounds);
* T8192 x batch 16, 9q/3kv, head dim 64, RGBA 4x4 V;
* a ragged batch of 64 sequences of U[512, 16384] tokens, 32q/8kv, head dim
  128, 4-bit group-32 K and scalar 6x6 V in 96-token pages with block tables
  (default tile: about twelve rounds of workgroups).

Each checks that every output is finite, that permuting the batch permutes
the outputs bit for bit (each sequence is computed independently of its
position), and compares two or three sequences with the oracle (rtol 1e-3 /
atol 2e-3 against fp32 NumPy attention on V decoded by the oracle, relative L2
<= 1e-4 against FP64). V is encoded at low effort (quality 10) to keep the
host-side setup short; the decode is exercised the same way.
"""
import time

import numpy as np
import pytest

from oracle import attention_ref as R

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

RTOL, ATOL, REL_L2 = 1e-3, 2e-3, 1e-4


@pytest.fixture(scope="module")
def gpu():
    from astc_kv import gpu as G
    G.lib()
    return G


def _contiguous(gpu, b, hq, hkv, t, d, block, heavy, seed):
    from astc_kv.atlas import Atlas, build_atlas
    from astc_kv.gpu import DeviceAtlas
    from test_gpu_attention import oracle_v
    t0 = time.time()
    rng = np.random.default_rng(seed)
    q = rng.normal(size=(b, hq, d)).astype(np.float32)
    k = (rng.standard_t(3, size=(b, hkv, t, d)) if heavy else rng.normal(size=(b, hkv, t, d))).astype(np.float16)
    v = rng.normal(0, 0.5, size=(b, hkv, t, d)).astype(np.float32)
    atlas = build_atlas(v, "rgba", block, page_tokens=120 if block[1] == 5 else 128, quality=10)
    del v
    print(f"T{t} b{b} {hq}q/{hkv}kv D{d} RGBA {block}: encoded in {time.time() - t0:.1f}s", flush=True)
    dev = DeviceAtlas.from_host(atlas)
    qt, kt = torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda()
    params = gpu.make_params(dev, hq)
    print(f"default tile {params.tile_tokens}, {params.splits} splits", flush=True)
    out = gpu.decode_attention(qt, kt, dev, params=params).cpu().numpy()
    assert np.isfinite(out).all()
    perm = rng.permutation(b)
    dev_p = DeviceAtlas(dev.blocks[perm].contiguous(), dev.scale[perm].contiguous(), dev.offset[perm].contiguous(),
                        t, d, "rgba", block[0], block[1], dev.page_tokens)
    out_p = gpu.decode_attention(qt[perm].contiguous(), kt[perm].contiguous(), dev_p, params=params).cpu().numpy()
    assert np.array_equal(out_p, out[perm])
    for i in (0, b - 1):
        small = Atlas(atlas.blocks[i:i + 1], atlas.scale[i:i + 1], atlas.offset[i:i + 1], t, d, "rgba", *block,
                      atlas.page_tokens)
        vi = oracle_v(small)
        ref = R.decode_attention(q[i:i + 1], k[i:i + 1].astype(np.float32), vi)
        np.testing.assert_allclose(out[i:i + 1], ref, rtol=RTOL, atol=ATOL, err_msg=f"sequence {i}")
        assert R.relative_l2(R.attention_fp64(q[i], k[i].astype(np.float64), vi[0]), out[i]) <= REL_L2
    return params


def test_t32768_b8_32q8kv_d128_rgba4x4(gpu):
    params = _contiguous(gpu, 8, 32, 8, 32768, 128, (4, 4), True, 32768)
    assert params.tile_tokens == 2048 and params.splits == 16


def test_t8192_b16_9q3kv_d64_rgba4x4(gpu):
    _contiguous(gpu, 16, 9, 3, 8192, 64, (4, 4), False, 8192)


def test_ragged64_d128_u4k_scalar6x6_paged(gpu):
    from astc_kv.paged import build_paged
    from oracle.paged_ref import host_kv
    t0 = time.time()
    rng = np.random.default_rng(20261202)
    lens = rng.integers(512, 16384 + 1, size=64).tolist()
    k, v = [], []
    for t in lens:
        kk = rng.normal(size=(8, t, 128)).astype(np.float32)
        kk[..., :4] *= 8.0
        k.append(kk.astype(np.float16))
        v.append(rng.normal(0.0, 0.5, size=(8, t, 128)).astype(np.float32))
    pk = build_paged(k, v, "scalar", (6, 6), 96, quality=10, k_format="u4g32", tail=False, seed=7)
    del k, v
    print(f"ragged 64 x U[512,16384] ({sum(lens)} tokens): built in {time.time() - t0:.1f}s", flush=True)
    cache = gpu.DevicePagedKV.from_host(pk)
    q = rng.normal(size=(64, 32, 128)).astype(np.float32)
    qt = torch.from_numpy(q).cuda()
    params = gpu.paged_params(cache, 32)
    print(f"default tile {params.tile_tokens}, {params.splits} splits at most", flush=True)
    assert params.tile_tokens == 720
    out = gpu.paged_decode_attention(qt, cache, params=params).cpu().numpy()
    assert np.isfinite(out).all()
    perm = rng.permutation(64)
    cache.block_table.copy_(cache.block_table[torch.from_numpy(perm).cuda()].clone())
    cache.seq_lens.copy_(cache.seq_lens[torch.from_numpy(perm).cuda()].clone())
    out_p = gpu.paged_decode_attention(qt[torch.from_numpy(perm).cuda()].contiguous(), cache,
                                       params=params).cpu().numpy()
    assert np.array_equal(out_p, out[perm])
    for i in (int(np.argmin(lens)), int(np.argmax(lens)), 17):
        ki, vi = host_kv(pk, i)
        ref = R.decode_attention(q[i:i + 1], ki[None], vi[None])[0]
        np.testing.assert_allclose(out[i], ref, rtol=RTOL, atol=ATOL, err_msg=f"sequence {i}")
        assert R.relative_l2(R.attention_fp64(q[i], ki.astype(np.float64), vi), out[i]) <= REL_L2
