"""Representation layer of ASTC-KV: range normalisation, ASTC image layouts, the
codec round trip, byte accounting and the CPU reference numerics.

Drop-in for the reference's astc_kv/codec.py (same names, arguments, return
values and exceptions; citations per function). Two additive extensions:
`config["block"]` may be an (bx, by) pair for rectangular footprints such as
6x5, and `AstcEncoder` accepts `block=(bx, by)`. The codec behind
`AstcEncoder` is libakv_astc.so (include/astc_kv.h): this package's own C++
ASTC LDR encoder and decoder in place of the reference's astcenc binding.
"""
from __future__ import annotations

import ctypes as ct
import math
import struct
import time
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

_LIB_NAME = "libakv_astc.so"


def align(n: int, a: int) -> int:
    """Round n up to a multiple of a (astc_kv/codec.py:18-19)."""
    return -(-n // a) * a


def _footprint(block) -> tuple[int, int]:
    if isinstance(block, (tuple, list)):
        bx, by = (int(v) for v in block)
    else:
        bx = by = int(block)
    return bx, by


def load_codec_library(path: Path | None = None):
    """Load libakv_astc.so from next to this file and declare its signatures."""
    path = Path(path) if path else Path(__file__).with_name(_LIB_NAME)
    lib = ct.CDLL(str(path))
    lib.akv_create.argtypes = [ct.c_uint, ct.c_uint, ct.c_float, ct.c_int, ct.POINTER(ct.c_int)]
    lib.akv_create.restype = ct.c_void_p
    lib.akv_destroy.argtypes = [ct.c_void_p]
    lib.akv_error.argtypes = [ct.c_int]
    lib.akv_error.restype = ct.c_char_p
    lib.akv_encode.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_uint, ct.c_uint, ct.c_void_p, ct.c_size_t]
    lib.akv_decode.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_size_t, ct.c_void_p, ct.c_uint, ct.c_uint]
    lib.akv_encode_blocks.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_size_t, ct.c_void_p]
    lib.akv_decode_blocks_fp16.argtypes = [ct.c_uint, ct.c_uint, ct.c_void_p, ct.c_size_t, ct.c_void_p, ct.c_void_p]
    lib.akv_block_classes.argtypes = [ct.c_uint, ct.c_uint, ct.c_void_p, ct.c_size_t, ct.c_void_p]
    return lib


class AstcEncoder:
    """ASTC round trip through the akv_* bridge (astc_kv/codec.py:22-67).

    `block` is an int (square footprint, as in the reference) or (bx, by)."""

    def __init__(self, block, quality: float = 98, hdr: bool = False):
        self.lib = load_codec_library()
        self.ctx = None
        bx, by = _footprint(block)
        error = ct.c_int()
        self.ctx = self.lib.akv_create(bx, by, quality, int(hdr), ct.byref(error))
        self._check(error.value)
        if not self.ctx:
            raise RuntimeError("astc context allocation failed")
        self.block = block
        self.block_x, self.block_y = bx, by

    def _check(self, code: int):
        if code:
            raise RuntimeError(self.lib.akv_error(code).decode())

    def payload_bytes(self, width: int, height: int) -> int:
        return math.ceil(width / self.block_x) * math.ceil(height / self.block_y) * 16

    def roundtrip(self, image: np.ndarray) -> tuple[bytes, np.ndarray, float]:
        """Encode then decode one HxWx4 float image; returns (payload, decoded, encode seconds)."""
        image = np.ascontiguousarray(image, dtype=np.float32)
        h, w, comps = image.shape
        if comps != 4 or not np.isfinite(image).all():
            raise ValueError("Expected finite HxWx4 input")
        payload = np.empty(self.payload_bytes(w, h), np.uint8)
        decoded = np.empty_like(image)
        start = time.perf_counter()
        self._check(self.lib.akv_encode(self.ctx, image.ctypes.data, w, h, payload.ctypes.data, payload.size))
        seconds = time.perf_counter() - start
        self._check(self.lib.akv_decode(self.ctx, payload.ctypes.data, payload.size, decoded.ctypes.data, w, h))
        if not np.isfinite(decoded).all():
            raise ValueError("Non-finite ASTC reconstruction")
        return payload.tobytes(), decoded, seconds

    def encode_blocks(self, texels: np.ndarray) -> np.ndarray:
        """float32 [n, by, bx, 4] texels -> uint8 [n, 16] blocks."""
        texels = np.ascontiguousarray(texels, dtype=np.float32)
        n = texels.shape[0]
        if texels.shape[1:] != (self.block_y, self.block_x, 4):
            raise ValueError("Expected [n, by, bx, 4] texels")
        out = np.empty((n, 16), np.uint8)
        self._check(self.lib.akv_encode_blocks(self.ctx, texels.ctypes.data, n, out.ctypes.data))
        return out

    def close(self):
        if getattr(self, "ctx", None):
            self.lib.akv_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        self.close()


def fp16_floor(x):
    """Largest float16 <= x, elementwise (astc_kv/codec.py:70-74)."""
    x = np.asarray(x, np.float32)
    h = x.astype(np.float16)
    step_down = h.astype(np.float32) > x
    return np.where(step_down, np.nextafter(h, np.float16(-np.inf)), h).astype(np.float16)


def fp16_ceil(x):
    """Smallest float16 >= x, elementwise (astc_kv/codec.py:77-81)."""
    x = np.asarray(x, np.float32)
    h = x.astype(np.float16)
    step_up = h.astype(np.float32) < x
    return np.where(step_up, np.nextafter(h, np.float16(np.inf)), h).astype(np.float16)


@dataclass
class EncodedTensor:
    """One encoded [H,T,D] tensor (astc_kv/codec.py:84-113)."""
    decoded: np.ndarray
    payloads: list[bytes]
    width: int
    height: int
    block: object
    layout: str
    profile: str
    normalization: str
    offsets: np.ndarray
    scales: np.ndarray | None
    page_tokens: int
    byte_counts: dict[str, int]
    encode_cpu_s: float
    permutation: str | None = None
    metadata: dict = field(default_factory=dict)

    @property
    def logical_bytes(self):
        return sum(self.byte_counts.values())

    @property
    def bits_per_scalar(self):
        return self.logical_bytes * 8 / self.decoded.size

    def astc_file(self, head: int) -> bytes:
        """.astc container: magic, bx, by, bz=1, u24 width, height, depth=1, payload."""
        bx, by = _footprint(self.block)
        dims = b"".join(v.to_bytes(3, "little") for v in (self.width, self.height, 1))
        return struct.pack("<I", 0x5CA1AB13) + bytes((bx, by, 1)) + dims + self.payloads[head]


def _range_normalize(work, normalization, heads, tokens, dim, width, bx, by, page_tokens):
    """Returns (normalised values, offsets, scales) (astc_kv/codec.py:155-174)."""
    f32 = np.float32
    if normalization == "page_channel":
        pages = tokens // page_tokens
        grouped = work.reshape(heads, pages, page_tokens, dim)
        offset = fp16_floor(grouped.min(axis=2))
        spread = grouped.max(axis=2) - offset.astype(f32)
        scale = fp16_ceil(np.maximum(spread, f32(2 ** -24)))
        unit = (grouped - offset[:, :, None, :].astype(f32)) / scale[:, :, None, :].astype(f32)
        return unit.reshape(work.shape), offset, scale
    if normalization == "token":
        offset = fp16_floor(work.min(-1, keepdims=True))
        spread = work.max(-1, keepdims=True) - offset.astype(f32)
        scale = fp16_ceil(np.maximum(spread, f32(2 ** -24)))
        return (work - offset.astype(f32)) / scale.astype(f32), offset, scale
    if normalization == "block_min":
        padded = np.pad(work, ((0, 0), (0, 0), (0, width - dim)), mode="edge")
        tiles = padded.reshape(heads, tokens // by, by, width // bx, bx)
        offset = fp16_floor(tiles.min(axis=(2, 4)))
        unit = tiles - offset[:, :, None, :, None].astype(f32)
        return unit.reshape(heads, tokens, width), offset, None
    raise ValueError("Unknown normalization")


def encode_tensor(x: np.ndarray, config: dict, page_tokens: int = 96,
                  quality: float = 98, seed: int = 20261028) -> EncodedTensor:
    """Encode completed pages of an [H,T,D] tensor (astc_kv/codec.py:116-215).

    config: block (int or (bx, by)), layout "scalar"|"rgba", normalization
    "token"|"page_channel"|"block_min", optional profile and permutation."""
    x = np.asarray(x, np.float32)
    if x.ndim != 3 or not np.isfinite(x).all():
        raise ValueError("Expected finite [H,T,D]")
    heads, tokens, dim = x.shape
    bx, by = _footprint(config["block"])
    layout = config["layout"]
    profile = config.get("profile", "ldr")
    normalization = config["normalization"]
    permutation = config.get("permutation")
    if page_tokens % by:
        raise ValueError("Page boundary must align to ASTC block rows")
    if layout not in ("scalar", "rgba") or (layout == "rgba" and dim % 4):
        raise ValueError("Unsupported scalar/component layout")
    if tokens % page_tokens:
        raise ValueError("Only completed pages enter encoder; keep incomplete page in tail")
    if profile == "hdr" and (layout != "scalar" or normalization != "block_min"):
        raise ValueError("HDR pilot supports scalar block-min only")
    lanes = 1 if layout == "scalar" else 4
    width, height = align(dim // lanes, bx), tokens
    rng = np.random.default_rng(seed)
    token_order = np.arange(tokens)
    channel_order = np.arange(dim)
    map_bytes = 0
    if permutation == "tokens_within_page":
        within = rng.permutation(page_tokens)
        token_order = (np.arange(tokens // page_tokens)[:, None] * page_tokens + within[None]).ravel()
        map_bytes = page_tokens * 2
    elif permutation == "channels":
        channel_order = rng.permutation(dim)
        map_bytes = dim * 2
    elif permutation is not None:
        raise ValueError("Unknown permutation")
    work = x[:, token_order, :][:, :, channel_order]
    normalized, offset, scale = _range_normalize(work, normalization, heads, tokens, dim, width, bx, by,
                                                 page_tokens)
    if not np.isfinite(offset).all() or (scale is not None and not np.isfinite(scale).all()):
        raise ValueError("FP16 metadata overflow")
    if profile == "ldr":
        if normalized.min() < -1e-5 or normalized.max() > 1 + 1e-5:
            raise AssertionError("FP16 rounded metadata fails range coverage")
        normalized = np.clip(normalized, 0, 1)
    images = pack_images(normalized, layout, width)
    encoder = AstcEncoder((bx, by), quality, profile == "hdr")
    payloads, decoded, elapsed = [], [], 0.0
    try:
        for image in images:
            payload, dec, seconds = encoder.roundtrip(image)
            payloads.append(payload)
            decoded.append(dec)
            elapsed += seconds
    finally:
        encoder.close()
    rec = unpack_images(np.stack(decoded), layout, dim)
    if normalization == "block_min":
        tiles = np.stack(decoded)[..., 0].reshape(heads, height // by, by, width // bx, bx)
        rec = (tiles + offset[:, :, None, :, None].astype(np.float32)).reshape(heads, height, width)[:, :, :dim]
    elif normalization == "page_channel":
        pages = tokens // page_tokens
        grouped = rec.reshape(heads, pages, page_tokens, dim)
        rec = (grouped * scale[:, :, None, :].astype(np.float32) + offset[:, :, None, :].astype(np.float32))
        rec = rec.reshape(heads, tokens, dim)
    else:
        rec = rec * scale.astype(np.float32) + offset.astype(np.float32)
    rec = rec[:, np.argsort(token_order), :][:, :, np.argsort(channel_order)]
    counts = {"astc_blocks_including_edge_padding": sum(len(p) for p in payloads),
              "fp16_offsets": offset.nbytes, "fp16_scales": 0 if scale is None else scale.nbytes,
              "permutation_map": map_bytes}
    block_field = config["block"] if not isinstance(config["block"], list) else tuple(config["block"])
    return EncodedTensor(np.ascontiguousarray(rec), payloads, width, height, block_field, layout, profile,
                         normalization, offset, scale, page_tokens, counts, elapsed, permutation,
                         {"quality": quality, "original_scalars": x.size, "file_header_bytes": 16 * heads,
                          "logical_bytes_scope": "blocks+metadata+fixed_permutation; no allocation/staging/tail"})


def pack_images(normalized: np.ndarray, layout: str, width: int) -> np.ndarray:
    """[H,T,D] values in [0,1] -> RGBA images [H,T,width,4] (codec.py:181-187).

    scalar: texel (x=c, y=t) holds (u, u, u, 1); rgba: texel (x=c//4, y=t)
    holds channels 4x..4x+3. Columns beyond the tensor repeat the last one."""
    heads, tokens, dim = normalized.shape
    if layout == "scalar":
        grey = np.pad(normalized, ((0, 0), (0, 0), (0, width - dim)), mode="edge")
        images = np.ones((heads, tokens, width, 4), np.float32)
        images[..., :3] = grey[..., None]
        return images
    quads = normalized.reshape(heads, tokens, dim // 4, 4)
    return np.pad(quads, ((0, 0), (0, 0), (0, width - dim // 4), (0, 0)), mode="edge").astype(np.float32)


def unpack_images(images: np.ndarray, layout: str, dim: int) -> np.ndarray:
    """Inverse of pack_images for decoded images -> [H,T,D] normalised values."""
    if layout == "scalar":
        return images[..., :dim, 0]
    heads, tokens = images.shape[:2]
    return images[:, :, : dim // 4, :].reshape(heads, tokens, dim)


def affine_quantize(x: np.ndarray, bits: int, axis: str = "token", group: int = 64):
    """Affine uniform quantiser with bit-packed byte accounting
    (astc_kv/codec.py:218-250). Returns (CPU reconstruction, byte counts)."""
    dec, counts, *_ = affine_quantize_codes(x, bits, axis, group)
    return dec, counts


def affine_quantize_codes(x: np.ndarray, bits: int, axis: str = "token", group: int = 64):
    """affine_quantize plus its codes, packed bytes, fp16 offsets and scales.

    Codes are round-half-even of (x - o)/s clipped to [0, 2^bits - 1]; element i
    of each run of 8/bits codes sits at bit offset (i mod 8/bits)*bits."""
    x = np.asarray(x, np.float32)
    h, t, d = x.shape
    if bits not in (2, 4, 8):
        raise ValueError("Supported bit widths: 2,4,8")
    if axis == "token":
        if d % group:
            raise ValueError("group must divide channels")
        groups, reduce_axis = x.reshape(h, t, d // group, group), -1
    elif axis == "channel":
        if t % group:
            raise ValueError("group must divide tokens")
        groups, reduce_axis = x.reshape(h, t // group, group, d), 2
    else:
        raise ValueError("Unknown quantization axis")
    top = (1 << bits) - 1
    offset = fp16_floor(groups.min(axis=reduce_axis, keepdims=True))
    o32 = offset.astype(np.float32)
    scale = fp16_ceil(np.maximum((groups.max(axis=reduce_axis, keepdims=True) - o32) / top, np.float32(2 ** -24)))
    s32 = scale.astype(np.float32)
    codes = np.clip(np.rint((groups - o32) / s32), 0, top).astype(np.uint8)
    per_byte = 8 // bits
    flat = codes.ravel()
    flat = np.pad(flat, (0, (-flat.size) % per_byte))
    lanes = flat.reshape(-1, per_byte).astype(np.uint32) << (np.arange(per_byte, dtype=np.uint32) * bits)
    packed = np.bitwise_or.reduce(lanes, axis=1).astype(np.uint8)
    dec = (codes.astype(np.float32) * s32 + o32).reshape(x.shape)
    counts = {"packed_codes": packed.nbytes, "fp16_offsets": offset.nbytes, "fp16_scales": scale.nbytes}
    return dec, counts, codes, packed, offset, scale


def attention(q, k, v, positions):
    """GQA softmax attention for arbitrary query positions (astc_kv/codec.py:253-267).

    q [Hq,N,D], k/v [Hkv,T,D]; returns (out [Hq,N,D], p [Hq,N,T]) in float32."""
    hq, n, d = q.shape
    hk, t, kd = k.shape
    if v.shape != k.shape or kd != d or hq % hk:
        raise ValueError("Incompatible attention shapes")
    group = hq // hk
    grouped = np.asarray(q, np.float32).reshape(hk, group, n, d)
    keys_t = np.asarray(k, np.float32)[:, None].swapaxes(-1, -2)
    logits = np.matmul(grouped, keys_t) * np.float32(d ** -0.5)
    visible = np.arange(t)[None, :] <= np.asarray(positions)[:, None]
    logits = np.where(visible[None, None], logits, np.float32(-np.inf))
    logits -= logits.max(-1, keepdims=True)
    probs = np.exp(logits)
    probs /= probs.sum(-1, keepdims=True)
    out = np.matmul(probs, np.asarray(v, np.float32)[:, None]).reshape(hq, n, d)
    return out, probs.reshape(hq, n, t)


def errors(reference, estimate):
    """MSE, relative L2, max |err| and cosine (astc_kv/codec.py:270-274)."""
    a = np.asarray(reference, np.float64)
    b = np.asarray(estimate, np.float64)
    diff = b - a
    na, nb = np.linalg.norm(a.ravel()), np.linalg.norm(b.ravel())
    return {"mse": float(np.mean(diff * diff)),
            "relative_l2": float(np.linalg.norm(diff.ravel()) / max(na, 1e-30)),
            "max_abs": float(np.max(np.abs(diff))),
            "cosine": float(np.sum(a * b) / max(na * nb, 1e-30))}


def attention_metrics(reference, estimate, reference_probs, estimate_probs):
    """errors() plus KL and total variation of the probabilities (codec.py:277-283)."""
    metrics = errors(reference, estimate)
    a = np.asarray(reference_probs, np.float64)
    b = np.asarray(estimate_probs, np.float64)
    kl = np.sum(a * (np.log(np.maximum(a, 1e-300)) - np.log(np.maximum(b, 1e-300))), axis=-1)
    metrics.update(mean_kl_nats=float(np.mean(kl)), p95_kl_nats=float(np.percentile(kl, 95)),
                   mean_total_variation=float(np.mean(np.abs(a - b).sum(-1) * 0.5)))
    return metrics
