"""nimbus_amd: Nimbus's paged-attention hot path, rebuilt for AMD MI355X (gfx950).

Public drop-ins (same call signatures as Nimbus):

  nimbus_amd.kernels.cache_ops.write_kv                     reference.py:14-23
  nimbus_amd.kernels.paged_attention.paged_decode_attention paged_attention.py:101
  nimbus_amd.kernels.prefill_attention.build_programs       prefill_attention.py:81
  nimbus_amd.kernels.prefill_attention.paged_prefill_attention  prefill_attention.py:93
  nimbus_amd.model.attention.AttnMetadata / AttentionBackend    model/attention.py:24-95
  nimbus_amd.graphs.DecodeAttentionGraphs                   cuda_graph.py capture contract

All compute runs in libnimbus_attn.so (hand-written HIP kernels, C ABI in
include/nimbus_attn.h); build it with `python -m nimbus_amd.build`.
"""

__all__ = ["kernels", "model", "graphs", "workloads"]
