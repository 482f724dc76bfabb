"""MI355X (gfx950) HiFloat8 static W8A8KV8 hot path.

Modules:
  native    operator API (static_quant, soft_linear, soft_static_fused_linear, scaled_decode)
  scheme    static W8A8 linear method (input_scale / weight / weight_scale)
  kv_cache  paged HiF8 KV layout, fused static cache write, paged decode attention
  _build    in-tree build of libhif8_rocm.so and the torch extension
"""

__all__ = ["kv_cache", "native", "scheme"]
