"""MI355X (gfx950) drop-in for the per-frame decode path of EstudioCanciones.

kernels   -- int8_mm, rms, _rope_cache, _attn, _attn_combine, _silu_mul (app/kernels.py API)
engine    -- Linear, fuse, Emb, Block, Stack, HeartMuLaLite (app/engine.py API)
quant     -- q8_rows on the GPU (app/convert_final.py) and synthetic int8 weights
build     -- compiles csrc/*.hip into _lib/libecdecode.so (the C ABI of include/ecdecode.h)
"""
__version__ = "0.1.0"
