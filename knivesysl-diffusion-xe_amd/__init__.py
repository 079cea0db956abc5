"""MI355X (gfx950) fused layer kernels for the DiffusionGemma W4A16 MoE.

Drop-in modules, named after the reference's kernel modules:
  fused_rmsnorm    fused_rmsnorm, _fused_forward, patch_rmsnorms
  fused_moe_w4     moe_align (GPU routing metadata), fused_moe_w4 (the v1 path, any act_fn)
  fused_moe_w4_v2  fused_moe_w4_v2 (W4A16 128-expert fused MoE forward), moe_align_cuda (int32 align),
                   enable_ns_down, preshuffle_T_dn (the MOE_NS down pack)
  pack_experts     fused_experts_forward, packed_experts_forward, repack_experts (load-time repack),
                   GU_GS, DN_GS, pack_experts_module, pack_all_experts (quantise bf16 experts in place),
                   dump_moe_stats
  w4a16            quantize_w4, dequant_w4 (GPU W4 group quantisation and its inverse)
  load_w4          bind_expert_shards (one shared tensor per layer from experts_*.safetensors)
  layer            moe_layer: RMSNorm followed by the MoE forward
  router           router_forward, patch_routers (the expert router, the step before)
  moe_block        moe_block_forward, layer_forward, patch_moe_blocks (the MoE branch
                   with the layer's tail fused into the combine, the step after)
  fused_sampler_ops  fused_entropy, gumbel_argmax_sample, sample_step (the per-step sampler pass)
  fast_sampler     install, uninstall, stats (the generation-loop patches)
All compute runs in libksl.so (hand-written HIP, C ABI in include/ksl.h).
"""
from . import _lib
from .fused_moe_w4 import fused_moe_w4, moe_align
from .fused_moe_w4_v2 import enable_ns_down, fused_moe_w4_v2, moe_align_cuda, preshuffle_T_dn
from .fused_rmsnorm import fused_rmsnorm, patch_rmsnorms
from .fused_sampler_ops import fused_entropy, gumbel_argmax_sample, sample_step
from .pack_experts import (dump_moe_stats, fused_experts_forward, pack_all_experts, pack_experts_module,
                           packed_experts_forward, repack_experts)
from .w4a16 import dequant_w4, quantize_w4
from .load_w4 import bind_expert_shards
from .moe_block import layer_forward, moe_block_forward, patch_moe_blocks
from .router import patch_routers, router_forward

__all__ = ["fused_rmsnorm", "patch_rmsnorms", "moe_align", "moe_align_cuda", "fused_moe_w4", "fused_moe_w4_v2",
           "enable_ns_down", "preshuffle_T_dn", "fused_experts_forward", "packed_experts_forward", "repack_experts",
           "pack_experts_module", "pack_all_experts", "dump_moe_stats", "quantize_w4", "dequant_w4", "bind_expert_shards",
           "router_forward", "patch_routers", "moe_block_forward", "layer_forward", "patch_moe_blocks",
           "fused_entropy", "gumbel_argmax_sample", "sample_step"]
