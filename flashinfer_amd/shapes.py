"""Problem shapes the native library is compiled for.

The kernels take the hidden size H and the expert intermediate size I as
compile-time constants (as the reference hard-codes them, kernel.py:615-625);
each (H, I) gets its own library. Routing (256 experts in 8 groups, top-4
groups, top-8), the 32 local experts and the 128-element scale blocks are
those of the ds-routing definition family and stay fixed.

Supported: H a multiple of 1024, I a multiple of 256.
"""
DEFAULT_SHAPE = (7168, 2048)  # moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048
SHAPES = (DEFAULT_SHAPE, (4096, 1536))


def supported(H: int, I: int) -> bool:
    return H > 0 and I > 0 and H % 1024 == 0 and I % 256 == 0


def lib_name(H: int, I: int) -> str:
    return "libmi_moe.so" if (H, I) == DEFAULT_SHAPE else f"libmi_moe_h{H}_i{I}.so"
