"""Paged, ragged decode attention (akv_hip_paged_decode_attention) against the
NumPy oracle, per sequence, on K and V reconstructed on the host from the
pages each block-table row names: FP16 or 4-bit K (code * scale + offset in
float32, astc_kv/codec.py:248), V restored from the oracle's decode of the
page blocks plus the FP16 tail. Tolerance as test_gpu_attention: rtol 1e-3 /
atol 2e-3 against the fp32 oracle, relative L2 <= 1e-4 against FP64."""
import numpy as np
import pytest

from oracle import attention_ref as R
from oracle.paged_ref import host_kv

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

RTOL, ATOL, REL_L2 = 1e-3, 2e-3, 1e-4


@pytest.fixture(scope="module")
def gpu():
    from astc_kv import gpu as G
    G.lib()
    return G


CASES = [
    # layout, block, page, dim, hq, hkv, k_format, tail
    ("scalar", (6, 6), 96, 128, 8, 2, "u4g32", True),
    ("rgba", (4, 4), 64, 128, 8, 2, "fp16", False),
    ("rgba", (6, 5), 80, 64, 9, 3, "fp16", True),
    ("scalar", (6, 6), 96, 64, 9, 3, "u4g32", True),
    ("rgba", (8, 8), 64, 64, 8, 1, "u4g32", False),
    # scalar at head dim 128 (three workgroups per CU, one tile per group)
    # with the other GQA group sizes and FP16 K
    ("scalar", (6, 6), 96, 128, 3, 3, "fp16", True),     # G = 1
    ("scalar", (6, 6), 96, 128, 6, 3, "u4g32", False),   # G = 2
    ("scalar", (6, 6), 48, 128, 9, 3, "u4g32", True),    # G = 3
    ("scalar", (6, 6), 96, 128, 16, 2, "fp16", False),   # G = 8
]


@pytest.mark.parametrize("layout,block,page,d,hq,hkv,kf,tail", CASES)
def test_paged_attention(gpu, layout, block, page, d, hq, hkv, kf, tail):
    from astc_kv.paged import build_paged
    rng = np.random.default_rng(page + d + hq)
    lens = [100, 517, 1200, page, 333, 1]
    k = []
    for t in lens:
        kk = rng.normal(size=(hkv, t, d))
        kk[..., :4] *= 8.0
        k.append(kk.astype(np.float16))
    v = [rng.normal(0, 0.5, size=(hkv, t, d)).astype(np.float32) for t in lens]
    pk = build_paged(k, v, layout, block, page, quality=20, k_format=kf, tail=tail, seed=len(lens))
    cache = gpu.DevicePagedKV.from_host(pk)
    q = rng.normal(size=(len(lens), hq, d)).astype(np.float32)
    qt = torch.from_numpy(q).cuda()
    step = 16
    while step % block[1]:
        step += 16
    for tile in (None, 2 * step):
        out = gpu.paged_decode_attention(qt, cache, tile=tile).cpu().numpy()
        for i in range(len(lens)):
            ki, vi = host_kv(pk, i)
            ref = R.decode_attention(q[i:i + 1], ki[None], vi[None])[0]
            np.testing.assert_allclose(out[i], ref, rtol=RTOL, atol=ATOL, err_msg=f"sequence {i} tile {tile}")
            ref64 = R.attention_fp64(q[i], ki.astype(np.float64), vi)
            assert R.relative_l2(ref64, out[i]) <= REL_L2


def test_long_splits_many_chunks(gpu):
    """Splits of thousands of tokens: block rows far from the split's first page
    (more than 255 rows, past the range of the 24-bit quotient helper)."""
    from astc_kv.paged import build_paged
    rng = np.random.default_rng(31)
    lens = [3000, 2900, 97]
    k = [rng.normal(size=(2, t, 128)).astype(np.float16) for t in lens]
    v = [rng.normal(0, 0.5, size=(2, t, 128)).astype(np.float32) for t in lens]
    pk = build_paged(k, v, "scalar", (6, 6), 96, quality=20, k_format="u4g32", tail=False, seed=1)
    cache = gpu.DevicePagedKV.from_host(pk)
    q = rng.normal(size=(len(lens), 8, 128)).astype(np.float32)
    out = gpu.paged_decode_attention(torch.from_numpy(q).cuda(), cache, tile=2880).cpu().numpy()
    for i in range(len(lens)):
        ki, vi = host_kv(pk, i)
        ref = R.decode_attention(q[i:i + 1], ki[None], vi[None])[0]
        np.testing.assert_allclose(out[i], ref, rtol=RTOL, atol=ATOL, err_msg=f"sequence {i}")


APPEND_CASES = [
    # layout, block, page, dim, hkv, k_format
    ("scalar", (6, 6), 96, 128, 2, "u4g32"),
    ("rgba", (6, 5), 80, 64, 3, "fp16"),
    ("rgba", (4, 4), 64, 64, 2, "u4g32"),
]


@pytest.mark.parametrize("layout,block,page,d,hkv,kf", APPEND_CASES)
def test_append_matches_scratch_build(gpu, layout, block, page, d, hkv, kf):
    """Token-by-token appends (akv_hip_paged_append, with the pages they
    complete encoded on the host and committed by akv_hip_paged_commit_pages)
    leave exactly the pools build_paged makes from the whole sequences: K (4-bit
    codes and fp16 offset/scale computed on the GPU), V blocks, scale/offset and
    tail, bit for bit, and the same decode output. V is fp16-valued, as the
    tail keeps it."""
    from astc_kv.paged import build_paged
    P = page
    print(f"append case {layout} {block} P{P} D{d} {kf}", flush=True)
    rng = np.random.default_rng(P + d)
    start = [P - 2, 2 * P - 1, 3, P, 1]
    A = P + 3                              # every sequence completes at least one page
    full = [t + A for t in start]
    k = [rng.normal(size=(hkv, t, d)).astype(np.float32) * np.float32(3) for t in full]
    v = [rng.normal(0, 0.5, size=(hkv, t, d)).astype(np.float16).astype(np.float32) for t in full]
    spare = 2 * P
    pk0 = build_paged([x[:, :t] for x, t in zip(k, start)], [x[:, :t] for x, t in zip(v, start)], layout, block, P,
                      quality=20, k_format=kf, tail=True, seed=7, reserve_tokens=A + spare)
    ref = build_paged(k, v, layout, block, P, quality=20, k_format=kf, tail=True, seed=7, reserve_tokens=spare)
    assert np.array_equal(pk0.block_table, ref.block_table)   # the same page assignment
    cache = gpu.DevicePagedKV.from_host(pk0)
    completed = 0
    for j in range(A):
        kn = torch.from_numpy(np.stack([x[:, t + j] for x, t in zip(k, start)])).cuda()
        vn = torch.from_numpy(np.stack([x[:, t + j] for x, t in zip(v, start)])).cuda()
        completed += len(cache.append(kn, vn, quality=20))
    assert completed == sum((t + A) // P - t // P for t in start)
    assert cache.lens == full and cache.seq_lens.cpu().tolist() == full
    assert np.array_equal(cache.k_pages.cpu().numpy(), ref.k_pages)
    if kf == "u4g32":
        assert np.array_equal(cache.k_meta.cpu().numpy(), ref.k_meta)
    assert np.array_equal(cache.v_blocks.cpu().numpy(), ref.v_blocks)
    assert np.array_equal(cache.v_scale.cpu().numpy(), ref.v_scale)
    assert np.array_equal(cache.v_offset.cpu().numpy(), ref.v_offset)
    tail = cache.v_tail.cpu().numpy()
    for i, t in enumerate(full):
        assert np.array_equal(tail[i, :, :t % P], ref.v_tail[i, :, :t % P])
    q = torch.from_numpy(rng.normal(size=(len(full), 4 * hkv, d)).astype(np.float32)).cuda()
    out_a = gpu.paged_decode_attention(q, cache)
    out_b = gpu.paged_decode_attention(q, gpu.DevicePagedKV.from_host(ref))
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)


def test_append_needs_a_reserved_page(gpu):
    from astc_kv.paged import build_paged
    rng = np.random.default_rng(11)
    k = [rng.normal(size=(1, 64, 64)).astype(np.float16)]
    v = [rng.normal(0, 0.5, size=(1, 64, 64)).astype(np.float32)]
    cache = gpu.DevicePagedKV.from_host(build_paged(k, v, "rgba", (4, 4), 64, quality=10, tail=True))
    x = torch.zeros((1, 1, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="no page"):
        cache.append(x, x)
    assert cache.lens == [64]
