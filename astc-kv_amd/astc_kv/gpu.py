"""HIP decode attention on MI355X through libastckv_hip.so (include/astc_kv_hip.h).

PyTorch-ROCm provides device memory and the stream; every computation runs in
this package's hand-written gfx950 kernels. There is no CPU or PyTorch
fallback: if the library or a GPU is missing, the entry points raise.

Reference counterparts: the Metal host's dispatch of attention_split_gqa3 +
attention_merge (metal/probe_gqa_v10.mm:648-681) and its decode readbacks
(:258-274).
"""
from __future__ import annotations

import ctypes as ct
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from .atlas import Atlas, texel_columns

_LIB = None
LIB_PATH = Path(__file__).with_name("libastckv_hip.so")

LAYOUTS = {"scalar": 0, "rgba": 1}


class AkvAttnParams(ct.Structure):
    _fields_ = [(name, ct.c_uint32) for name in (
        "batch", "tokens", "query_heads", "kv_heads", "dim", "page_tokens", "tile_tokens", "splits",
        "layout", "block_x", "block_y", "atlas_rows", "atlas_cols")]


class AkvPagedParams(ct.Structure):
    _fields_ = [(name, ct.c_uint32) for name in (
        "batch", "max_tokens", "query_heads", "kv_heads", "dim", "page_tokens", "max_pages", "num_pages",
        "tile_tokens", "splits", "layout", "block_x", "block_y", "atlas_cols", "k_format")]


K_FORMATS = {"fp16": 0, "u4g32": 1}


def lib():
    """Load the HIP extension; raises if it is absent or no GPU is visible."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python astc-kv_amd/build.py`")
        if not torch.cuda.is_available():
            raise RuntimeError("astc_kv.gpu needs a ROCm GPU (torch.cuda.is_available() is False)")
        L = ct.CDLL(str(LIB_PATH))
        P = ct.POINTER(AkvAttnParams)
        vp = ct.c_void_p
        L.akv_hip_decode_attention.argtypes = [P, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.akv_hip_decode_attention_fused.argtypes = [P, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.akv_hip_fp16_attention_fused.argtypes = [P, vp, vp, vp, vp, vp, vp, vp, vp]
        L.akv_hip_attention_split.argtypes = [P, vp, vp, vp, vp, vp, vp, vp, vp]
        L.akv_hip_attention_merge.argtypes = [P, vp, vp, vp, vp]
        L.akv_hip_fp16_attention.argtypes = [P, vp, vp, vp, vp, vp, vp, vp]
        L.akv_hip_decode_values.argtypes = [P, vp, vp, vp]
        L.akv_hip_decode_blocks.argtypes = [vp, ct.c_size_t, ct.c_uint, ct.c_uint, vp, vp]
        PP = ct.POINTER(AkvPagedParams)
        L.akv_hip_paged_decode_attention.argtypes = [PP] + [vp] * 14
        L.akv_hip_paged_task_tokens.argtypes = [PP]
        L.akv_hip_paged_task_tokens.restype = ct.c_int
        L.akv_hip_paged_append.argtypes = [PP] + [vp] * 8
        L.akv_hip_paged_commit_pages.argtypes = [PP, ct.c_uint32] + [vp] * 8
        L.akv_hip_task_tokens.argtypes = [P, ct.c_int]
        L.akv_hip_task_tokens.restype = ct.c_int
        L.akv_hip_error_string.argtypes = [ct.c_int]
        L.akv_hip_error_string.restype = ct.c_char_p
        for f in ("akv_hip_decode_attention", "akv_hip_attention_split", "akv_hip_attention_merge",
                  "akv_hip_fp16_attention", "akv_hip_decode_values", "akv_hip_decode_blocks",
                  "akv_hip_paged_decode_attention", "akv_hip_paged_append", "akv_hip_paged_commit_pages"):
            getattr(L, f).restype = ct.c_int
        _LIB = L
    return _LIB


def _check(rc: int):
    if rc:
        raise RuntimeError(f"libastckv_hip: {lib().akv_hip_error_string(rc).decode()} (code {rc})")


def _stream(device) -> ct.c_void_p:
    return ct.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None):
    return ct.c_void_p(t.data_ptr()) if t is not None else None


def _need(t: torch.Tensor, dtype, name: str, shape=None):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


def task_tokens(params: AkvAttnParams, astc: bool = True) -> int:
    """Tokens per chunk (the unit a workgroup decodes and attends at once)."""
    rc = lib().akv_hip_task_tokens(ct.byref(params), int(astc))
    if rc <= 0:
        _check(rc if rc < 0 else -2)
    return rc


def default_tile(batch: int, kv_heads: int, tokens: int, chunk: int, block: int = 1, cu_count: int = 256,
                 groups_per_cu: int = 3, overhead_tokens: int = 64) -> int:
    """Tokens per split (a multiple of `block`: 16 for the kernels here).

    * Fewer chunks than CUs: splits of about tokens * batch * kv_heads / CUs
      tokens (at least 16) for parallelism, but at most 32 splits per
      sequence (the merge reads every split's state; the reference's scalar
      6x6 payload at batch 1: T2048 19.2 us with 32 splits, 20.8 us with 16;
      T384 17.9 us with 24); above 64 tokens, whole groups of four tiles
      (multiples of 64).
    * Up to 32 rounds of one-chunk workgroups (groups_per_cu per CU): the
      tile (at most 16 chunks) minimising rounds x (tile + overhead_tokens),
      i.e. the time of the last workgroup to finish when each costs its tokens
      plus a fixed overhead (a partial last round idles most CUs); among tiles
      within 3% of that minimum, the fewest splits, then the lowest cost.
      (T32768 batch 8, 8 KV heads, D128: 16 chunks of 128 per split, two
      rounds, 397 us; 8 chunks, four rounds, 407 us.)
    * More: several chunks per split (up to 16, about two rounds or more),
      which also cuts the split-state traffic; the tail is small there."""
    seqs = batch * kv_heads
    slots = groups_per_cu * cu_count
    total = seqs * -(-tokens // chunk)
    if total < cu_count:
        want = max(16, -(-tokens * seqs // cu_count), -(-tokens // 32))
        step = 64 if want > 64 else block
        return min(chunk, -(-want // step) * step)
    if total <= 32 * slots:
        top = min(16 * chunk, -(-tokens // block) * block)
        tiles = range(top - top % block, 0, -block)
        cost = {t: -(-seqs * -(-tokens // t) // slots) * (t + overhead_tokens) for t in tiles}
        floor = min(cost.values())
        # Within 3% of the best, fewer workgroups win (less fixed work), then
        # the lower cost (the shortest tile for that many splits).
        near = [t for t in tiles if cost[t] <= 1.03 * floor]
        fewest = min(-(-tokens // t) for t in near)
        return min((cost[t], -t) for t in near if -(-tokens // t) == fewest)[1] * -1
    per_split = max(1, min(16, total // (2 * slots)))
    return per_split * chunk


def tile_for_splits(tokens: int, splits: int, block_y: int, dim: int) -> int:
    """Tile giving exactly `splits` splits when possible (e.g. T2048 in 8
    splits): ceil(tokens / splits), rounded up to 16 tokens when that keeps the
    split count (16-token splits are the kernel's natural grain; any tile is
    accepted)."""
    tile = -(-tokens // splits)
    t16 = -(-tile // 16) * 16
    return t16 if -(-tokens // t16) == splits else tile


@dataclass
class DeviceAtlas:
    """An Atlas resident in GPU memory."""
    blocks: torch.Tensor    # uint8 [B, Hkv, rows, cols, 16]
    scale: torch.Tensor     # float16 [B, Hkv, T]
    offset: torch.Tensor    # float16 [B, Hkv, T]
    tokens: int
    dim: int
    layout: str
    block_x: int
    block_y: int
    page_tokens: int

    @classmethod
    def from_host(cls, atlas: Atlas, device="cuda") -> "DeviceAtlas":
        return cls(torch.from_numpy(np.ascontiguousarray(atlas.blocks)).to(device),
                   torch.from_numpy(np.ascontiguousarray(atlas.scale)).to(device),
                   torch.from_numpy(np.ascontiguousarray(atlas.offset)).to(device),
                   atlas.tokens, atlas.dim, atlas.layout, atlas.block_x, atlas.block_y, atlas.page_tokens)

    @property
    def batch(self) -> int:
        return self.blocks.shape[0]

    @property
    def kv_heads(self) -> int:
        return self.blocks.shape[1]

    def clone(self) -> "DeviceAtlas":
        return DeviceAtlas(self.blocks.clone(), self.scale.clone(), self.offset.clone(), self.tokens, self.dim,
                           self.layout, self.block_x, self.block_y, self.page_tokens)

    def nbytes(self) -> int:
        return self.blocks.numel() + 2 * self.scale.numel() + 2 * self.offset.numel()


def make_params(atlas: DeviceAtlas, query_heads: int, tile: int | None = None) -> AkvAttnParams:
    b, h = atlas.batch, atlas.kv_heads
    cols = -(-texel_columns(atlas.dim, atlas.layout) // atlas.block_x)
    if atlas.blocks.shape[3] != cols:
        raise ValueError("atlas columns do not match dim/layout/footprint")

    def build(t):
        return AkvAttnParams(b, atlas.tokens, query_heads, h, atlas.dim, atlas.page_tokens, t,
                             -(-atlas.tokens // t), LAYOUTS[atlas.layout], atlas.block_x, atlas.block_y,
                             atlas.blocks.shape[2], cols)

    if tile is None:
        whole = -(-atlas.tokens // 16) * 16   # one split: the chunk is not clipped
        # Resident workgroups per CU: three at head dim 64, two at 128 (registers).
        tile = default_tile(b, h, atlas.tokens, task_tokens(build(whole)), 16,
                            groups_per_cu=3 if atlas.dim == 64 else 2)
    return build(tile)


def _check_qk(q: torch.Tensor, k: torch.Tensor, b: int, h: int, t: int, d: int):
    if q.dim() != 3 or q.shape[0] != b or q.shape[2] != d or q.shape[1] % h:
        raise ValueError(f"q must be [B={b}, Hq, D={d}] with Hq a multiple of {h}")
    _need(q, torch.float32, "q")
    _need(k, torch.float16, "k", (b, h, t, d))


def attention_split(q, k, atlas: DeviceAtlas, params: AkvAttnParams, partial=None, stats=None):
    """Split pass only; returns (partial [B,Hq,S,D], stats [B,Hq,S,2])."""
    b, hq, d = q.shape
    _check_qk(q, k, atlas.batch, atlas.kv_heads, atlas.tokens, atlas.dim)
    s = params.splits
    if partial is None:
        partial = torch.empty((b, hq, s, d), dtype=torch.float32, device=q.device)
    if stats is None:
        stats = torch.empty((b, hq, s, 2), dtype=torch.float32, device=q.device)
    _check(lib().akv_hip_attention_split(ct.byref(params), _ptr(q), _ptr(k), _ptr(atlas.blocks),
                                         _ptr(atlas.scale), _ptr(atlas.offset), _ptr(partial), _ptr(stats),
                                         _stream(q.device)))
    return partial, stats


def attention_merge(params: AkvAttnParams, partial, stats, out=None):
    b, hq, s, d = partial.shape
    if out is None:
        out = torch.empty((b, hq, d), dtype=torch.float32, device=partial.device)
    _check(lib().akv_hip_attention_merge(ct.byref(params), _ptr(partial), _ptr(stats), _ptr(out),
                                         _stream(partial.device)))
    return out


_ARRIVALS: dict = {}


def arrivals(device, count: int) -> torch.Tensor:
    """Zeroed per-(sequence, kv head) counters for the one-launch entry points,
    cached per device. Every call leaves them zero; calls that may run
    concurrently (different streams) need their own tensors."""
    device = torch.device(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), count)
    t = _ARRIVALS.get(key)
    if t is None:
        t = _ARRIVALS[key] = torch.zeros(count, dtype=torch.int32, device=device)
    return t


def decode_attention(q: torch.Tensor, k: torch.Tensor, atlas: DeviceAtlas, tile: int | None = None,
                     params: AkvAttnParams | None = None, return_states: bool = False, partial=None, stats=None,
                     out=None, fused: bool = True):
    """One decode step: q [B,Hq,D] f32, k [B,Hkv,T,D] f16, V from the ASTC atlas.
    Returns out [B,Hq,D] f32 (and (partial, stats) if return_states). fused:
    one launch (the last split workgroup of a kv head merges); otherwise the
    split and merge passes."""
    if params is None:
        params = make_params(atlas, q.shape[1], tile)
    if not fused:
        partial, stats = attention_split(q, k, atlas, params, partial, stats)
        out = attention_merge(params, partial, stats, out)
        return (out, partial, stats) if return_states else out
    b, hq, d = q.shape
    _check_qk(q, k, atlas.batch, atlas.kv_heads, atlas.tokens, atlas.dim)
    s = params.splits
    if partial is None:
        partial = torch.empty((b, hq, s, d), dtype=torch.float32, device=q.device)
    if stats is None:
        stats = torch.empty((b, hq, s, 2), dtype=torch.float32, device=q.device)
    if out is None:
        out = torch.empty((b, hq, d), dtype=torch.float32, device=q.device)
    _check(lib().akv_hip_decode_attention_fused(ct.byref(params), _ptr(q), _ptr(k), _ptr(atlas.blocks),
                                                _ptr(atlas.scale), _ptr(atlas.offset), _ptr(partial), _ptr(stats),
                                                _ptr(out), _ptr(arrivals(q.device, b * atlas.kv_heads)),
                                                _stream(q.device)))
    return (out, partial, stats) if return_states else out


def fp16_params(batch, kv_heads, query_heads, tokens, dim, tile=None, cu_count: int = 256) -> AkvAttnParams:
    """The FP16 control streams 16-token tiles per wave, so its default split is
    about one round of 3 resident workgroups per CU (at least 64 tokens)."""
    def build(t):
        return AkvAttnParams(batch, tokens, query_heads, kv_heads, dim, 0, t, -(-tokens // t), 0, 0, 0, 0, 0)

    if tile is None:
        splits = max(1, -(-3 * cu_count // (batch * kv_heads)))
        tile = max(64, -(-(-(-tokens // splits)) // 16) * 16)
    return build(tile)


def fp16_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tile: int | None = None,
                   params: AkvAttnParams | None = None, partial=None, stats=None, out=None, fused: bool = True):
    """FP16-K/V control: same schedule, V read as restored fp16 [B,Hkv,T,D];
    fused as in decode_attention."""
    b, hkv, t, d = k.shape
    _check_qk(q, k, b, hkv, t, d)
    _need(v, torch.float16, "v", (b, hkv, t, d))
    if params is None:
        params = fp16_params(b, hkv, q.shape[1], t, d, tile)
    s = params.splits
    if partial is None:
        partial = torch.empty((b, q.shape[1], s, d), dtype=torch.float32, device=q.device)
    if stats is None:
        stats = torch.empty((b, q.shape[1], s, 2), dtype=torch.float32, device=q.device)
    if out is None:
        out = torch.empty((b, q.shape[1], d), dtype=torch.float32, device=q.device)
    arr = arrivals(q.device, b * hkv) if fused else None
    _check(lib().akv_hip_fp16_attention_fused(ct.byref(params), _ptr(q), _ptr(k), _ptr(v), _ptr(partial),
                                              _ptr(stats), _ptr(out), _ptr(arr), _stream(q.device)))
    return out


def decode_values(atlas: DeviceAtlas, tile: int | None = None) -> torch.Tensor:
    """Normalised V as the attention kernel decodes it: float16 [B,Hkv,T,D]."""
    params = make_params(atlas, atlas.kv_heads, tile)
    u = torch.empty((atlas.batch, atlas.kv_heads, atlas.tokens, atlas.dim), dtype=torch.float16,
                    device=atlas.blocks.device)
    _check(lib().akv_hip_decode_values(ct.byref(params), _ptr(atlas.blocks), _ptr(u), _stream(u.device)))
    return u


def decode_blocks(blocks: torch.Tensor, block_x: int, block_y: int) -> torch.Tensor:
    """uint8 [n,16] ASTC blocks -> float16 RGBA texels [n, by, bx, 4]."""
    _need(blocks, torch.uint8, "blocks")
    n = blocks.numel() // 16
    out = torch.empty((n, block_y, block_x, 4), dtype=torch.float16, device=blocks.device)
    _check(lib().akv_hip_decode_blocks(_ptr(blocks), n, block_x, block_y, _ptr(out), _stream(blocks.device)))
    return out


# --- paged, ragged batches -----------------------------------------------------

@dataclass
class DevicePagedKV:
    """A PagedKV (astc_kv.paged) resident in GPU memory."""
    k_pages: torch.Tensor
    k_meta: torch.Tensor | None
    v_blocks: torch.Tensor
    v_scale: torch.Tensor
    v_offset: torch.Tensor
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    v_tail: torch.Tensor | None
    lens: list
    dim: int
    layout: str
    block_x: int
    block_y: int
    page_tokens: int
    k_format: str
    table_host: np.ndarray | None = None   # host copy of block_table (page ids for append/commit)

    @classmethod
    def from_host(cls, pk, device="cuda") -> "DevicePagedKV":
        def dev(a):
            return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device)
        return cls(dev(pk.k_pages), dev(pk.k_meta), dev(pk.v_blocks), dev(pk.v_scale), dev(pk.v_offset),
                   dev(pk.block_table), dev(pk.seq_lens), dev(pk.v_tail), pk.seq_lens.tolist(), pk.dim, pk.layout,
                   pk.block_x, pk.block_y, pk.page_tokens, pk.k_format, np.array(pk.block_table))

    @property
    def batch(self) -> int:
        return len(self.lens)

    @property
    def kv_heads(self) -> int:
        return self.k_pages.shape[1]

    def pool_params(self) -> AkvPagedParams:
        """The pool fields of AkvPagedParams (append and commit use no others)."""
        return AkvPagedParams(self.batch, max(self.lens), self.kv_heads, self.kv_heads, self.dim, self.page_tokens,
                              self.block_table.shape[1], self.k_pages.shape[0], 0, 0, LAYOUTS[self.layout],
                              self.block_x, self.block_y, self.v_blocks.shape[3], K_FORMATS[self.k_format])

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, quality: float = 50, threads: int | None = None):
        """Append one token per sequence (k_new, v_new f32 [B, Hkv, D] on the
        GPU) with akv_hip_paged_append and advance the lengths. Each page this
        completes is encoded on the host from its FP16 tail (astc_kv.atlas, the
        encoder build_paged uses) and copied into its V pool page with one
        akv_hip_paged_commit_pages launch. Returns the sequences whose page
        completed."""
        if self.v_tail is None:
            raise ValueError("appending needs the FP16 tail (build_paged(tail=True))")
        shape = (self.batch, self.kv_heads, self.dim)
        _need(k_new, torch.float32, "k_new", shape)
        _need(v_new, torch.float32, "v_new", shape)
        P = self.page_tokens
        for i, n in enumerate(self.lens):
            pg = n // P
            if pg >= self.table_host.shape[1] or not 0 <= int(self.table_host[i, pg]) < self.k_pages.shape[0]:
                raise ValueError(f"sequence {i} has no page for token {n} (reserve pages in build_paged)")
        params = self.pool_params()
        dev = k_new.device
        _check(lib().akv_hip_paged_append(ct.byref(params), _ptr(k_new), _ptr(v_new), _ptr(self.k_pages),
                                          _ptr(self.k_meta), _ptr(self.block_table), _ptr(self.seq_lens),
                                          _ptr(self.v_tail), _stream(dev)))
        self.seq_lens += 1
        self.lens = [n + 1 for n in self.lens]
        done = [i for i, n in enumerate(self.lens) if n % P == 0]
        if done:
            from .atlas import build_atlas
            tails = self.v_tail[done].float().cpu().numpy()          # [n, Hkv, P, D]
            at = build_atlas(tails, self.layout, (self.block_x, self.block_y), P, quality, threads)
            ids = torch.tensor([int(self.table_host[i, self.lens[i] // P - 1]) for i in done], dtype=torch.int32,
                               device=dev)
            blocks = torch.from_numpy(np.ascontiguousarray(at.blocks)).to(dev)
            scale = torch.from_numpy(np.ascontiguousarray(at.scale)).to(dev)
            offset = torch.from_numpy(np.ascontiguousarray(at.offset)).to(dev)
            _check(lib().akv_hip_paged_commit_pages(ct.byref(params), len(done), _ptr(ids), _ptr(blocks), _ptr(scale),
                                                    _ptr(offset), _ptr(self.v_blocks), _ptr(self.v_scale),
                                                    _ptr(self.v_offset), _stream(dev)))
            torch.cuda.current_stream(dev).synchronize()   # staging buffers are freed on return
        return done


def paged_params(cache: DevicePagedKV, query_heads: int, tile: int | None = None, cu_count: int = 256) -> AkvPagedParams:
    """Tile default: about twelve rounds of resident workgroups over the whole
    ragged batch (in steps of lcm(16, block_y) tokens; with uneven lengths
    shorter splits balance the rounds), within the kernel's limit of 62 pages
    per split. (64 sequences of U[512,16384] tokens, 8 KV heads, D128: 720
    tokens, 2.39 ms; six rounds, 1392 tokens: 2.46 ms.)"""
    P, by = cache.page_tokens, cache.block_y
    step = 16
    while step % by:
        step += 16
    max_t = max(cache.lens)
    if tile is None:
        groups = (3 if cache.dim == 64 else 2) * cu_count
        want = -(-sum(cache.lens) * cache.kv_heads // (12 * groups))
        tile = max(step, -(-want // step) * step)
        limit = (62 * P) // step * step
        while (tile + P) * P >= 1 << 24 and tile > step:
            limit -= step
            tile = min(tile, limit)
        tile = min(tile, limit, -(-max_t // step) * step)
        if tile < step or (tile + P) * P >= 1 << 24:
            raise ValueError(f"no legal split tile for page_tokens {P} (at most 4080 for 16-token steps)")
    cols = cache.v_blocks.shape[3]
    return AkvPagedParams(cache.batch, max_t, query_heads, cache.kv_heads, cache.dim, P, cache.block_table.shape[1],
                          cache.k_pages.shape[0], tile, -(-max_t // tile), LAYOUTS[cache.layout], cache.block_x,
                          by, cols, K_FORMATS[cache.k_format])


def paged_task_tokens(params: AkvPagedParams) -> int:
    rc = lib().akv_hip_paged_task_tokens(ct.byref(params))
    if rc < 0:
        _check(rc)
    return rc


def paged_decode_attention(q: torch.Tensor, cache: DevicePagedKV, params: AkvPagedParams | None = None,
                           tile: int | None = None, partial=None, stats=None, out=None,
                           return_states: bool = False):
    """One decode step over a ragged batch: q [B,Hq,D] f32 -> out [B,Hq,D] f32."""
    b, hq, d = q.shape
    if b != cache.batch or d != cache.dim or hq % cache.kv_heads:
        raise ValueError("q does not match the paged cache")
    _need(q, torch.float32, "q")
    if params is None:
        params = paged_params(cache, hq, tile)
    s = params.splits
    if partial is None:
        partial = torch.empty((b, hq, s, d), dtype=torch.float32, device=q.device)
    if stats is None:
        stats = torch.empty((b, hq, s, 2), dtype=torch.float32, device=q.device)
    if out is None:
        out = torch.empty((b, hq, d), dtype=torch.float32, device=q.device)
    _check(lib().akv_hip_paged_decode_attention(
        ct.byref(params), _ptr(q), _ptr(cache.k_pages), _ptr(cache.k_meta), _ptr(cache.v_blocks),
        _ptr(cache.v_scale), _ptr(cache.v_offset), _ptr(cache.block_table), _ptr(cache.seq_lens),
        _ptr(cache.v_tail), _ptr(partial), _ptr(stats), _ptr(out), _ptr(arrivals(q.device, b * cache.kv_heads)),
        _stream(q.device)))
    return (out, partial, stats) if return_states else out
