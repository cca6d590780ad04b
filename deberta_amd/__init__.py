"""deberta_amd — MI355X-native fused disentangled self-attention (DeBERTa-v2/v3).

Public surface:
  DisentangledSelfAttention   drop-in module (reference forward signature)
  disentangled_attention      functional op on projected layers
  build_relative_position, make_log_bucket_position, relative_offset_table
  normalize_keep_mask, build_doc_block_mask, get_attention_mask
  SegmentMask                 packed-document ids in place of the dense mask
  FusedSelfOutput, FusedOutput, FusedIntermediate, FusedRTDHead,
  RelativeEmbeddings          the blocks around the attention on fused row
                              kernels (residual + LayerNorm, bias + GELU,
                              classifier + BCE loss)
  normalize_attention_kernel  the attention-kernel selector
The compute runs in libdsa.so (hand-written HIP for gfx950) through the
torch.library ops ``deberta_amd::dsa_fwd`` / ``deberta_amd::dsa_bwd``.
"""

from deberta_amd.attention import DisentangledSelfAttention, disentangled_attention, fused_attention
from deberta_amd.blocks import (
    FusedIntermediate,
    FusedOutput,
    FusedRTDHead,
    FusedSelfOutput,
    RelativeEmbeddings,
    fused_add_layer_norm,
)
from deberta_amd.config import normalize_attention_kernel, normalize_pos_att_type
from deberta_amd.masks import SegmentMask, build_doc_block_mask, get_attention_mask, normalize_keep_mask
from deberta_amd.relpos import build_relative_position, make_log_bucket_position, relative_offset_table

__all__ = [
    "DisentangledSelfAttention",
    "disentangled_attention",
    "fused_attention",
    "normalize_attention_kernel",
    "normalize_pos_att_type",
    "SegmentMask",
    "build_doc_block_mask",
    "get_attention_mask",
    "normalize_keep_mask",
    "build_relative_position",
    "make_log_bucket_position",
    "relative_offset_table",
    "FusedSelfOutput",
    "FusedOutput",
    "FusedIntermediate",
    "FusedRTDHead",
    "RelativeEmbeddings",
    "fused_add_layer_norm",
]
