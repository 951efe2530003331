"""ASTC-KV for AMD Instinct MI355X (gfx950): ASTC-compressed V cache, software
ASTC decode fused into split-K decode attention.

astc_kv.codec  drop-in representation layer (reference astc_kv/codec.py)
astc_kv.atlas  compact block atlas: token-normalised V -> ASTC blocks on the GPU
astc_kv.gpu    HIP decode-attention entry points (libastckv_hip.so)
"""
__version__ = "0.1.0"
