"""ORACLE — test infrastructure only (tests/, __graft_entry__.smoke(), bench.py's
CPU-baseline leg). Never imported by the product package.

NumPy restatements of the reference's numerics on the decode-attention path:

* `attention`            astc_kv/codec.py:253-267   (fp32 GQA softmax attention)
* `attention_fp64`       metal/probe_gqa_v10.mm:345-369 (FP64 host reference)
* `relative_l2`          metal/probe_gqa_v10.mm:370-383 (the 1e-4 gate metric)
* `restore_token`        astc_kv/codec.py:206          (u*s + o, unfused fp32)
* `restore_page_channel` astc_kv/codec.py:203
* `split_states`/`merge` metal/attention_gqa_v10.metal:101-253 (split-K states and
                          their exact merge), in float64
* `fp16_floor/fp16_ceil` astc_kv/codec.py:70-81
* `normalize_token`      astc_kv/codec.py:162-166, :175-180
* `affine_quantize`      astc_kv/codec.py:218-250 (pinned by outputs of the reference
                          module itself, tests/golden/gen_affine_quantize.py)
* `normalize_token` is pinned by the reference's captured normalisation
  (scripts/probe_block_geometry.py:142-155 -> tests/golden/geometry/*_fixed_input.npz)
"""
from __future__ import annotations

import numpy as np


def fp16_floor(x):
    x = np.asarray(x, np.float32)
    h = x.astype(np.float16)
    return np.where(h.astype(np.float32) > x, np.nextafter(h, np.float16(-np.inf)), h).astype(np.float16)


def fp16_ceil(x):
    x = np.asarray(x, np.float32)
    h = x.astype(np.float16)
    return np.where(h.astype(np.float32) < x, np.nextafter(h, np.float16(np.inf)), h).astype(np.float16)


def normalize_token(x):
    """Token range normalisation: returns (u clipped to [0,1], offset f16, scale f16)."""
    x = np.asarray(x, np.float32)
    lo, hi = x.min(-1, keepdims=True), x.max(-1, keepdims=True)
    offset = fp16_floor(lo)
    scale = fp16_ceil(np.maximum(hi - offset.astype(np.float32), np.float32(2 ** -24)))
    u = (x - offset.astype(np.float32)) / scale.astype(np.float32)
    return np.clip(u, 0, 1), offset, scale


def restore_token(u, scale, offset):
    """fl32(fl32(u*s)+o): NumPy evaluates the multiply and the add separately."""
    u = np.asarray(u, np.float32)
    prod = u * np.asarray(scale, np.float32)
    return prod + np.asarray(offset, np.float32)


def restore_page_channel(u, scale, offset, page_tokens):
    """u [H,T,D], scale/offset [H,pages,D] -> [H,T,D]."""
    h, t, d = u.shape
    view = np.asarray(u, np.float32).reshape(h, t // page_tokens, page_tokens, d)
    rec = view * np.asarray(scale, np.float32)[:, :, None, :] + np.asarray(offset, np.float32)[:, :, None, :]
    return rec.reshape(h, t, d)


def attention(q, k, v, positions):
    """GQA attention output and probabilities for arbitrary query positions (fp32)."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    hq, n, d = q.shape
    hk, t, kd = k.shape
    if v.shape != k.shape or kd != d or hq % hk:
        raise ValueError("Incompatible attention shapes")
    qq = q.reshape(hk, hq // hk, n, d)
    scores = np.matmul(qq, k[:, None].swapaxes(-1, -2)) * np.float32(d ** -0.5)
    mask = np.arange(t)[None, :] <= np.asarray(positions)[:, None]
    scores = np.where(mask[None, None], scores, np.float32(-np.inf))
    scores -= scores.max(-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(-1, keepdims=True)
    out = np.matmul(p, v[:, None]).reshape(hq, n, d)
    return out, p.reshape(hq, n, t)


def attention_fp64(q, k, v):
    """Single query token per head, all keys visible, FP64 accumulation.
    q [Hq,D], k/v [Hkv,T,D] -> [Hq,D]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    hq, d = q.shape
    hk = k.shape[0]
    g = hq // hk
    out = np.empty((hq, d))
    for h in range(hq):
        s = k[h // g] @ q[h] / np.sqrt(d)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v[h // g]
    return out


def relative_l2(reference, estimate):
    a = np.asarray(reference, np.float64).ravel()
    b = np.asarray(estimate, np.float64).ravel()
    return float(np.linalg.norm(b - a) / max(np.linalg.norm(a), 1e-30))


def decode_attention(q, k, v):
    """The decode step the GPU path computes: one query token per (sequence, head)
    seeing every key. q [B,Hq,D], k/v [B,Hkv,T,D] (float) -> out [B,Hq,D] fp32,
    through the fp32 restatement of astc_kv/codec.py:253-267."""
    q = np.asarray(q, np.float32)
    out = np.empty(q.shape, np.float32)
    for b in range(q.shape[0]):
        t = k[b].shape[1]
        o, _ = attention(q[b][:, None, :], k[b], v[b], np.array([t - 1]))
        out[b] = o[:, 0, :]
    return out


def split_states(q, k, u, scale, offset, tile):
    """Per-split (m, l, acc) states of split-K decode attention in float64, with the
    factored token affine acc = sum p*s*u + sum p*o (attention_gqa_v10.metal:155-226).
    q [Hq,D]; k, u [Hkv,T,D]; scale/offset [Hkv,T]. Returns m [Hq,S], l [Hq,S],
    acc [Hq,S,D]; an empty split has m=-inf, l=0, acc=0."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    u = np.asarray(u, np.float64)
    scale = np.asarray(scale, np.float64)
    offset = np.asarray(offset, np.float64)
    hq, d = q.shape
    hk, t, _ = k.shape
    g = hq // hk
    splits = max(1, -(-t // tile))
    m = np.full((hq, splits), -np.inf)
    l = np.zeros((hq, splits))
    acc = np.zeros((hq, splits, d))
    for h in range(hq):
        kh = h // g
        for s in range(splits):
            lo, hi = s * tile, min(s * tile + tile, t)
            if lo >= hi:
                continue
            sc = k[kh, lo:hi] @ q[h] / np.sqrt(d)
            m[h, s] = sc.max()
            p = np.exp(sc - m[h, s])
            l[h, s] = p.sum()
            acc[h, s] = (p * scale[kh, lo:hi]) @ u[kh, lo:hi] + (p * offset[kh, lo:hi]).sum()
    return m, l, acc


def merge(m, l, acc):
    """Exact merge of split states (attention_gqa_v10.metal:229-253)."""
    mm = m.max(-1, keepdims=True)
    w = np.exp(m - mm)
    w[~np.isfinite(m)] = 0.0
    den = (l * w).sum(-1)
    return (acc * w[..., None]).sum(-2) / den[..., None]


def affine_quantize(x, bits, axis="token", group=64):
    """Restatement of astc_kv/codec.py:218-250: returns (decoded, counts, codes,
    packed, offset, scale). Codes are np.rint (half-to-even) of (x-o)/s,
    clipped to [0, 2^bits-1]; packing puts element i of each byte group at bit
    offset (i % (8/bits)) * bits."""
    x = np.asarray(x, np.float32)
    h, t, d = x.shape
    if bits not in (2, 4, 8):
        raise ValueError("Supported bit widths: 2,4,8")
    if axis == "token":
        if d % group:
            raise ValueError("group must divide channels")
        view = x.reshape(h, t, d // group, group)
        gax = -1
    elif axis == "channel":
        if t % group:
            raise ValueError("group must divide tokens")
        view = x.reshape(h, t // group, group, d)
        gax = 2
    else:
        raise ValueError("Unknown quantization axis")
    levels = (1 << bits) - 1
    offset = fp16_floor(view.min(axis=gax, keepdims=True))
    maximum = view.max(axis=gax, keepdims=True)
    scale = fp16_ceil(np.maximum((maximum - offset.astype(np.float32)) / levels, np.float32(2 ** -24)))
    code = np.clip(np.rint((view - offset.astype(np.float32)) / scale.astype(np.float32)), 0, levels).astype(np.uint8)
    flat = code.ravel()
    per = 8 // bits
    if flat.size % per:
        flat = np.pad(flat, (0, per - flat.size % per))
    packed = np.zeros(flat.size // per, np.uint8)
    for i in range(per):
        packed |= flat[i::per] << (i * bits)
    dec = (code.astype(np.float32) * scale.astype(np.float32) + offset.astype(np.float32)).reshape(x.shape)
    counts = {"packed_codes": packed.nbytes, "fp16_offsets": offset.nbytes, "fp16_scales": scale.nbytes}
    return dec, counts, code, packed, offset, scale
