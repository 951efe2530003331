"""GPU decode of blocks no encoder here produces, bit-exact against the oracle.

* The blocks the oracle reduction tests build (tests/test_oracle_reductions.py:
  every LDR endpoint mode, swapped and blue-contracted endpoints, bit
  transfer, mixed endpoint classes, dual plane, identity and reduced weight
  grids of several footprints) through akv_hip_decode_blocks.
* The same blocks plus 60,000 random 128-bit blocks per case (every block
  mode, dual plane, 4 partitions, void extent, error blocks) laid out as V
  atlases and decoded by the attention kernel's own header and texel code
  (akv_hip_decode_values): scalar and RGBA layouts at head dim 64 and 128,
  which run decode_header<1>, decode_header<4> and the D=128 variant that
  decodes only the weight groups below a block's weight count.
* Decode attention and paged decode attention over random V blocks against
  the oracle (tolerance as test_gpu_attention: rtol 1e-3 / atol 2e-3, relative
  L2 <= 1e-4 against FP64).
"""
import numpy as np
import pytest

from oracle import astc_oracle as O
from oracle import attention_ref as R

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

RTOL, ATOL, REL_L2 = 1e-3, 2e-3, 1e-4


@pytest.fixture(scope="module")
def gpu():
    from astc_kv import gpu as G
    G.lib()
    return G


def _constructed(bx, by):
    from test_oracle_reductions import constructed_blocks
    return constructed_blocks(bx, by)


def _random_blocks(seed, n):
    rng = np.random.default_rng(seed)
    blocks = rng.integers(0, 256, size=(n, 16), dtype=np.uint8)
    blocks[: n // 20, 0] = 0xFC              # void-extent selectors, valid and invalid extents
    blocks[: n // 20, 1] = (blocks[: n // 20, 1] & 0xF0) | 0x0D
    return blocks


@pytest.mark.parametrize("bx,by", [(6, 6), (4, 4), (5, 4), (6, 5), (8, 5), (8, 8), (10, 6)])
def test_constructed_blocks_decode_blocks(gpu, bx, by):
    blocks = _constructed(bx, by)
    print(f"{bx}x{by}: {len(blocks)} constructed blocks", flush=True)
    t = torch.from_numpy(np.array(blocks, np.uint8)).cuda()
    got = gpu.decode_blocks(t, bx, by).cpu().numpy().view(np.uint16)
    exp, kinds = O.decode_blocks_fp16(blocks, bx, by)
    assert np.all(kinds == 0)
    bad = np.flatnonzero((got != exp.view(np.uint16)).any(axis=(1, 2, 3)))
    assert bad.size == 0, f"{bad.size} blocks differ, first {blocks[bad[0]].tolist()}"


def _atlas(blocks, layout, bx, by, dim, seed=0):
    """A batch-1, one-kv-head Atlas whose blocks are `blocks` in row-major
    order (repeated to fill the last row), with random fp16 scale/offset."""
    from astc_kv.atlas import Atlas, texel_columns
    cols = -(-texel_columns(dim, layout) // bx)
    rows = -(-len(blocks) // cols)
    idx = np.arange(rows * cols) % len(blocks)
    arr = np.ascontiguousarray(blocks[idx].reshape(1, 1, rows, cols, 16))
    tokens = rows * by
    rng = np.random.default_rng(seed)
    scale = rng.uniform(0.5, 2, size=(1, 1, tokens)).astype(np.float16)
    offset = rng.uniform(-1, 1, size=(1, 1, tokens)).astype(np.float16)
    return Atlas(arr, scale, offset, tokens, dim, layout, bx, by, by)


def _oracle_u(atlas):
    b, h, r, c = atlas.blocks.shape[:4]
    tex, _ = O.decode_blocks_fp16(atlas.blocks.reshape(-1, 16), atlas.block_x, atlas.block_y)
    img = tex.reshape(b, h, r, c, atlas.block_y, atlas.block_x, 4).transpose(0, 1, 2, 4, 3, 5, 6)
    img = img.reshape(b, h, r * atlas.block_y, c * atlas.block_x, 4)[:, :, : atlas.tokens].astype(np.float32)
    if atlas.layout == "scalar":
        return np.ascontiguousarray(img[..., : atlas.dim, 0])
    return np.ascontiguousarray(img[:, :, :, : atlas.dim // 4].reshape(b, h, atlas.tokens, atlas.dim))


ATLAS_CASES = [("scalar", (6, 6), 64), ("scalar", (6, 6), 128), ("rgba", (6, 6), 64), ("rgba", (6, 6), 128),
               ("rgba", (6, 5), 64), ("rgba", (4, 4), 128), ("rgba", (4, 4), 64), ("scalar", (8, 8), 64)]


@pytest.mark.parametrize("layout,block,dim", ATLAS_CASES)
def test_attention_decode_stage_on_constructed_and_random_blocks(gpu, layout, block, dim):
    from astc_kv.gpu import DeviceAtlas
    bx, by = block
    blocks = np.concatenate([_constructed(bx, by), _random_blocks(bx * 100 + by + dim, 60000)])
    atlas = _atlas(blocks, layout, bx, by, dim)
    print(f"{layout} {bx}x{by} D{dim}: {atlas.tokens} tokens, {atlas.blocks.shape[2]} block rows", flush=True)
    dev = DeviceAtlas.from_host(atlas)
    expect = _oracle_u(atlas)
    for tile in (None, 48):
        got = gpu.decode_values(dev, tile).cpu().numpy().astype(np.float32)
        bad = np.argwhere(got.view(np.uint32) != expect.view(np.uint32))
        assert bad.size == 0, f"tile {tile}: {len(bad)} values differ, first (b, h, t, d) {bad[0].tolist()}"


@pytest.mark.parametrize("layout,block,dim,hq,hkv", [("rgba", (6, 5), 64, 9, 3), ("scalar", (6, 6), 128, 8, 2)])
def test_attention_over_random_blocks(gpu, layout, block, dim, hq, hkv):
    from astc_kv.atlas import Atlas, texel_columns
    from astc_kv.gpu import DeviceAtlas
    bx, by = block
    rng = np.random.default_rng(dim + hq)
    b, t = 2, 900
    cols = -(-texel_columns(dim, layout) // bx)
    rows = -(-t // by)
    blocks = _random_blocks(dim, b * hkv * rows * cols).reshape(b, hkv, rows, cols, 16)
    scale = rng.uniform(0.2, 1.5, size=(b, hkv, t)).astype(np.float16)
    offset = rng.uniform(-1, 1, size=(b, hkv, t)).astype(np.float16)
    atlas = Atlas(blocks, scale, offset, t, dim, layout, bx, by, by)
    v = R.restore_token(_oracle_u(atlas), scale.astype(np.float32)[..., None], offset.astype(np.float32)[..., None])
    q = rng.normal(size=(b, hq, dim)).astype(np.float32)
    k = rng.normal(size=(b, hkv, t, dim)).astype(np.float16)
    dev = DeviceAtlas.from_host(atlas)
    for tile in (None, 100):
        out = gpu.decode_attention(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), dev, tile).cpu().numpy()
        ref = R.decode_attention(q, k.astype(np.float32), v)
        np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL)
        for i in range(b):
            assert R.relative_l2(R.attention_fp64(q[i], k[i].astype(np.float64), v[i]), out[i]) <= REL_L2


def test_paged_attention_over_random_v_blocks(gpu):
    from astc_kv.paged import build_paged
    from oracle.paged_ref import host_kv
    rng = np.random.default_rng(77)
    lens = [700, 130, 1000, 96]
    k = [rng.normal(size=(2, t, 128)).astype(np.float16) for t in lens]
    v = [rng.normal(0, 0.5, size=(2, t, 128)).astype(np.float32) for t in lens]
    pk = build_paged(k, v, "scalar", (6, 6), 96, quality=10, k_format="u4g32", tail=True, seed=5)
    pk.v_blocks[...] = _random_blocks(5, pk.v_blocks.size // 16).reshape(pk.v_blocks.shape)
    cache = __import__("astc_kv.gpu", fromlist=["gpu"]).DevicePagedKV.from_host(pk)
    q = rng.normal(size=(len(lens), 8, 128)).astype(np.float32)
    out = gpu.paged_decode_attention(torch.from_numpy(q).cuda(), cache).cpu().numpy()
    for i in range(len(lens)):
        ki, vi = host_kv(pk, i)
        ref = R.decode_attention(q[i:i + 1], ki[None], vi[None])[0]
        np.testing.assert_allclose(out[i], ref, rtol=RTOL, atol=ATOL, err_msg=f"sequence {i}")


@pytest.mark.parametrize("layout,block,dim", [("scalar", (6, 6), 64), ("rgba", (6, 5), 64), ("rgba", (4, 4), 128),
                                              ("scalar", (6, 6), 128), ("scalar", (8, 8), 64)])
def test_fill_area_overflow(gpu, layout, block, dim):
    """An atlas of reduced-grid, one-plane blocks only (from the constructed
    and random blocks): every chunk has far more of them than the fill area's
    32 slots, so the fill stage and the compute path for the blocks past the
    last slot both run; the decode stays bit-exact against the oracle."""
    from astc_kv import codec
    from astc_kv.gpu import DeviceAtlas
    bx, by = block
    pool = np.concatenate([_constructed(bx, by), _random_blocks(bx * 7 + by + dim, 200000)])
    lib = codec.load_codec_library()
    cls = np.empty(len(pool), np.uint32)
    assert lib.akv_block_classes(bx, by, pool.ctypes.data, len(pool), cls.ctypes.data) == 0
    keep = ((cls & 3) == 0) & (((cls >> 4) & 1) == 0) & (((cls >> 5) & 1) == 0)
    blocks = pool[keep]
    assert len(blocks) > 2000
    atlas = _atlas(blocks, layout, bx, by, dim, seed=dim)
    print(f"{layout} {bx}x{by} D{dim}: {len(blocks)} reduced-grid blocks, {atlas.tokens} tokens", flush=True)
    dev = DeviceAtlas.from_host(atlas)
    expect = _oracle_u(atlas)
    for tile in (None, 48):
        got = gpu.decode_values(dev, tile).cpu().numpy().astype(np.float32)
        bad = np.argwhere(got.view(np.uint32) != expect.view(np.uint32))
        assert bad.size == 0, f"tile {tile}: {len(bad)} values differ, first (b, h, t, d) {bad[0].tolist()}"
