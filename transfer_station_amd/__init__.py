"""MI355X-native bf16 flash-attention forward behind the reference's C entry points.

The product is libattn_flash.so (HIP kernels for gfx950 + a C host layer); this package
is its Python host mirror (ctypes) and build recipe."""
from .attn import (ATTN_BK_DEFAULT, ATTN_BK_MAX, ATTN_BK_MIN, ATTN_D_MAX, ATTN_NOALLOC_D_MAX,
                   ATTN_NOALLOC_SCRATCH_BYTES, ATTN_SCRATCH_ALIGN, AttnTimes, DeviceBuffer, Event,
                   attn_flash, attn_flash_noalloc, attn_flash_pick_bk, attn_flash_plan,
                   attn_flash_scratch_bytes, device_count, device_info, get_stream,
                   pack_v_full, parse_plan, run_attention, set_stream, synchronize, synth_lcg_qkv,
                   synth_normal_bf16, synth_normal_qkv)

__all__ = [n for n in dir() if not n.startswith("_")]
