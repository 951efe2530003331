"""Drop-in boundary cases on the GPU.

* The reference's own correctness protocol for the GQA split kernel: T391 with
  tiles 1, 7, 13 and 256 (configs/gqa_v10_20261029.json:23-40; any tile is a
  legal Params.tile_tokens, probe_gqa_v10.mm:466), on its astcenc payloads,
  against its archived decode (v_decoded.f32) and the NumPy oracle.
* Any tile_tokens >= 1 on synthetic atlases (splits starting inside block rows).
* Paged calls with bad device-side metadata: a length past max_tokens, a
  zero length and page ids outside the pool leave every later call correct.

Tolerance as test_gpu_attention: rtol 1e-3 / atol 2e-3 against the fp32
oracle, relative L2 <= 1e-4 against FP64 (probe_gqa_v10.mm:719-725).
"""
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


def _check(out, q, k, v):
    ref = R.decode_attention(q, k.astype(np.float32), v)
    np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL)
    for b in range(q.shape[0]):
        assert R.relative_l2(R.attention_fp64(q[b], k[b].astype(np.float64), v[b]), out[b]) <= REL_L2


@pytest.mark.parametrize("tile", [1, 7, 13, 256])
def test_reference_correctness_cases_t391(gpu, golden, tile):
    from astc_kv.atlas import atlas_from_manifest
    from astc_kv.gpu import DeviceAtlas
    print(f"T391 tile {tile}", flush=True)
    d = golden / "t391"
    atlas, _ = atlas_from_manifest(d)
    q = np.fromfile(d / "q.f32", "<f4").reshape(1, 9, 64)
    k = np.fromfile(d / "k.f16", "<f2").reshape(1, 3, 391, 64)
    v_ref = np.fromfile(d / "v_decoded.f32", "<f4").reshape(1, 3, 391, 64)
    dev = DeviceAtlas.from_host(atlas)
    # Decode through the attention kernel's own decode stage with this tile:
    # u * s + o recomposes the reference's astcenc-decoded V bit for bit.
    u = gpu.decode_values(dev, tile).cpu().numpy().astype(np.float32)
    rec = R.restore_token(u, atlas.scale.astype(np.float32)[..., None], atlas.offset.astype(np.float32)[..., None])
    assert np.array_equal(rec.view(np.uint32), v_ref.view(np.uint32))
    qt, kt = torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda()
    params = gpu.make_params(dev, 9, tile)
    assert params.tile_tokens == tile and params.splits == -(-391 // tile)
    fused = gpu.decode_attention(qt, kt, dev, params=params).cpu().numpy()
    two = gpu.decode_attention(qt, kt, dev, params=params, fused=False).cpu().numpy()
    _check(fused, q, k, v_ref)
    _check(two, q, k, v_ref)


@pytest.mark.parametrize("layout,block,d,hq,hkv,tiles", [
    ("rgba", (6, 5), 64, 9, 3, (1, 5, 17, 100, 333)),
    ("scalar", (6, 6), 128, 8, 2, (3, 29, 250)),
    ("rgba", (8, 8), 64, 8, 8, (9, 71)),
])
def test_any_tile(gpu, layout, block, d, hq, hkv, tiles):
    from astc_kv.atlas import build_atlas
    from astc_kv.gpu import DeviceAtlas
    from test_gpu_attention import oracle_v, synthetic
    rng = np.random.default_rng(sum(tiles))
    q, k, v = synthetic(rng, 2, hq, hkv, 700, d)
    atlas = build_atlas(v, layout, block, page_tokens=120, quality=30)
    vr = oracle_v(atlas)
    dev = DeviceAtlas.from_host(atlas)
    qt, kt = torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda()
    for tile in tiles:
        print(f"{layout} {block} D{d} tile {tile}", flush=True)
        _check(gpu.decode_attention(qt, kt, dev, tile).cpu().numpy(), q, k, vr)


def _paged_case(gpu, rng):
    from astc_kv.paged import build_paged
    lens = [700, 130, 1000, 96]
    k = [rng.normal(size=(2, t, 64)).astype(np.float16) for t in lens]
    v = [rng.normal(0, 0.5, size=(2, t, 64)).astype(np.float32) for t in lens]
    pk = build_paged(k, v, "rgba", (6, 5), 80, quality=20, k_format="u4g32", tail=True, seed=3)
    q = rng.normal(size=(len(lens), 8, 64)).astype(np.float32)
    return pk, gpu.DevicePagedKV.from_host(pk), q


def _paged_ref(pk, q, i):
    from oracle.paged_ref import host_kv
    ki, vi = host_kv(pk, i)
    return R.decode_attention(q[i:i + 1], ki[None], vi[None])[0]


def test_paged_bad_lengths_then_good_call(gpu):
    """A device length past max_tokens reads as max_tokens (no split is left
    unmerged, so the arrival counters stay balanced); a zero length gives zeros.
    The following ordinary call matches the oracle."""
    rng = np.random.default_rng(41)
    pk, cache, q = _paged_case(gpu, rng)
    qt = torch.from_numpy(q).cuda()
    params = gpu.paged_params(cache, 8, tile=240)
    good = cache.seq_lens.clone()
    bad = good.clone()
    bad[1] = params.max_tokens + 500
    bad[3] = 0
    cache.seq_lens.copy_(bad)
    out_bad = gpu.paged_decode_attention(qt, cache, params=params).cpu().numpy()
    assert np.all(out_bad[3] == 0)
    for i in (0, 2):
        np.testing.assert_allclose(out_bad[i], _paged_ref(pk, q, i), rtol=RTOL, atol=ATOL)
    assert int(gpu.arrivals(qt.device, 4 * 2).abs().sum()) == 0
    cache.seq_lens.copy_(good)
    out = gpu.paged_decode_attention(qt, cache, params=params).cpu().numpy()
    for i in range(4):
        np.testing.assert_allclose(out[i], _paged_ref(pk, q, i), rtol=RTOL, atol=ATOL, err_msg=f"sequence {i}")


def test_paged_bad_page_ids_poison_only_their_sequence(gpu):
    """Block-table ids outside [0, num_pages) are read as page 0 and make that
    sequence's output NaN; the other sequences and the next call are exact."""
    rng = np.random.default_rng(43)
    pk, cache, q = _paged_case(gpu, rng)
    qt = torch.from_numpy(q).cuda()
    table = cache.block_table.clone()
    bad = table.clone()
    bad[0, 2] = -7
    bad[2, 0] = cache.k_pages.shape[0] + 3
    cache.block_table.copy_(bad)
    out_bad = gpu.paged_decode_attention(qt, cache).cpu().numpy()
    assert np.all(np.isnan(out_bad[0])) and np.all(np.isnan(out_bad[2]))
    for i in (1, 3):
        np.testing.assert_allclose(out_bad[i], _paged_ref(pk, q, i), rtol=RTOL, atol=ATOL)
    cache.block_table.copy_(table)
    out = gpu.paged_decode_attention(qt, cache).cpu().numpy()
    for i in range(4):
        np.testing.assert_allclose(out[i], _paged_ref(pk, q, i), rtol=RTOL, atol=ATOL, err_msg=f"sequence {i}")
