"""GPU decode parity: gfx950 ASTC decode vs the oracle, bit-exact.

* akv_hip_decode_blocks on the reference's astcenc payloads, on random 128-bit
  blocks for every supported footprint (all block modes, endpoint modes, dual
  plane, void-extent and error paths) and on one void-extent block per UNORM16
  value (exhaustive check of the FP16 conversion);
* akv_hip_decode_values, i.e. the attention kernel's own decode stage, on the
  fixture atlases and on synthetic RGBA / scalar atlases, against the oracle
  decode of the same blocks.
"""
import numpy as np
import pytest

from oracle import astc_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def gpu():
    from astc_kv import gpu as G
    G.lib()
    return G


def _gpu_decode(G, blocks: np.ndarray, bx, by):
    t = torch.from_numpy(np.ascontiguousarray(blocks, np.uint8).reshape(-1, 16)).cuda()
    out = G.decode_blocks(t, bx, by)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _compare(G, blocks, bx, by):
    got = _gpu_decode(G, blocks, bx, by).view(np.uint16)
    exp, _ = O.decode_blocks_fp16(blocks, bx, by)
    bad = np.argwhere((got != exp.view(np.uint16)).any(axis=(1, 2, 3)))
    assert bad.size == 0, f"{bx}x{by}: {bad.size} blocks differ, first {blocks[bad[0][0]].tolist()}"


def test_fixture_blocks(gpu, golden):
    blocks = [np.frombuffer(O.read_astc_file(p.read_bytes())["payload"], np.uint8)
              for p in sorted(golden.glob("t*/v-h*.astc"))]
    blocks += [np.fromfile(p, np.uint8) for p in sorted(golden.glob("geometry/*.bin"))]
    blocks += [np.fromfile(p, np.uint8) for p in sorted(golden.glob("holdout/*.bin"))]
    _compare(gpu, np.concatenate(blocks).reshape(-1, 16), 6, 6)


@pytest.mark.parametrize("bx,by", [(4, 4), (5, 4), (5, 5), (6, 5), (6, 6), (8, 5), (8, 6), (8, 8)])
def test_random_blocks(gpu, bx, by):
    rng = np.random.default_rng(bx * 16 + by)
    blocks = rng.integers(0, 256, size=(60000, 16), dtype=np.uint8)
    blocks[:3000, 0] = 0xFC              # void-extent selectors, valid and invalid extents
    blocks[:3000, 1] = (blocks[:3000, 1] & 0xF0) | 0x0D
    _compare(gpu, blocks, bx, by)


def test_unorm16_conversion_exhaustive(gpu):
    c = np.arange(65536, dtype=np.uint64)
    word = np.uint64(0x1FC | (3 << 10)) | (np.uint64((1 << 52) - 1) << np.uint64(12))
    lo = np.full(65536, word, np.uint64)
    hi = c | (c << np.uint64(16)) | (c << np.uint64(32)) | (c << np.uint64(48))
    blocks = np.stack([lo, hi], 1).view(np.uint8).reshape(-1, 16)
    got = _gpu_decode(gpu, blocks, 4, 4).view(np.uint16)
    expect = np.array([O.unorm16_to_fp16(int(v)) for v in range(65536)], np.uint16)
    assert np.array_equal(got[:, 0, 0, 0], expect)
    assert np.all(got == got[:, :1, :1, :1])


def _atlas_check(G, atlas, tile=None):
    from astc_kv.gpu import DeviceAtlas
    dev = DeviceAtlas.from_host(atlas)
    got = G.decode_values(dev, tile).cpu().numpy().astype(np.float32)
    expect = _oracle_normalized(atlas)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


def _oracle_normalized(atlas):
    b, h, r, c = atlas.blocks.shape[:4]
    tex, _ = O.decode_blocks_fp16(atlas.blocks.reshape(-1, 16), atlas.block_x, atlas.block_y)
    img = tex.reshape(b, h, r, c, atlas.block_y, atlas.block_x, 4).transpose(0, 1, 2, 4, 3, 5, 6)
    img = img.reshape(b, h, r * atlas.block_y, c * atlas.block_x, 4)[:, :, : atlas.tokens].astype(np.float32)
    if atlas.layout == "scalar":
        return np.ascontiguousarray(img[..., : atlas.dim, 0])
    return np.ascontiguousarray(img[:, :, :, : atlas.dim // 4].reshape(b, h, atlas.tokens, atlas.dim))


@pytest.mark.parametrize("name", ["t384", "t391"])
def test_decode_values_fixture(gpu, golden, name):
    from astc_kv.atlas import atlas_from_manifest
    atlas, _ = atlas_from_manifest(golden / name)
    for tile in (16, 48, 96, 256):
        _atlas_check(gpu, atlas, tile)


@pytest.mark.parametrize("layout,block,dim", [("rgba", (6, 5), 64), ("rgba", (4, 4), 64), ("rgba", (4, 4), 128),
                                              ("scalar", (6, 6), 64), ("rgba", (6, 6), 128), ("scalar", (8, 8), 64)])
def test_decode_values_synthetic(gpu, layout, block, dim):
    from astc_kv.atlas import build_atlas
    rng = np.random.default_rng(11)
    t = 500
    v = rng.normal(0, 0.5, size=(2, 2, t, dim)).astype(np.float32)
    atlas = build_atlas(v, layout, block, page_tokens=120 if block[1] != 8 else 120, quality=60)
    _atlas_check(gpu, atlas)
    _atlas_check(gpu, atlas, tile=48)
