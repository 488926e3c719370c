"""HIP kernels of the handoff, decode attention and the decode step, called through the C ABI."""
from .handoff import (pack_kv, pack_kv_batch, scatter_paged, scatter_paged_batch, gather_paged,
                      frame_shape, frame_views, stream_handle, validate_table, copy_kernel,
                      stream_probe, check_skipped)
from .attention import (decode_attention, decode_attention_rope, cache_append, greedy_argmax,
                        workspace_bytes, get_workspace, attn_read_probe)
from .decode_step import (rmsnorm, rope_cache_append, rope_cache_append_partials, swiglu, linear,
                          linear_swiglu, linear_argmax, linear_splitk, rmsnorm_partials,
                          linear_ssq, linear_swiglu_rms, fold_norm, linear_splitk_final, linear_splitk_rms,
                          linear_argmax_rms, row_ssq, embed_ssq, TiledWeight, tile_weight,
                          act_rows, act_tile, act_untile)

__all__ = ["pack_kv", "pack_kv_batch", "scatter_paged", "scatter_paged_batch", "gather_paged",
           "frame_shape", "frame_views", "stream_handle", "validate_table", "copy_kernel",
           "check_skipped",
           "stream_probe",
           "decode_attention", "decode_attention_rope", "cache_append", "greedy_argmax", "workspace_bytes", "get_workspace",
           "attn_read_probe",
           "rmsnorm", "rope_cache_append", "rope_cache_append_partials", "swiglu", "linear", "linear_swiglu", "linear_argmax",
           "linear_splitk", "rmsnorm_partials", "linear_ssq", "linear_swiglu_rms", "fold_norm",
           "linear_splitk_final", "linear_splitk_rms", "linear_argmax_rms", "row_ssq", "embed_ssq",
           "TiledWeight", "tile_weight", "act_rows", "act_tile", "act_untile"]
