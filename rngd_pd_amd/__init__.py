"""rngd_pd_amd: the rngd-pd prefill->decode KV handoff and decode_batch attention on MI355X.

Layers, in dependency order (each only imports the ones above it):
  _lib        ctypes binding of librngdpd.so (HIP kernels for gfx950, include/rngdpd.h)
  kernels     torch-facing wrappers: pack / scatter / gather / decode attention / argmax
  hip         streams, events, pinned staging buffers and same-GPU IPC handles
  connector   bf16 wire, Transport ABC + /dev/shm transport, frame codec,
              RngdKVConnector (the vLLM KVConnector surface)
  airm        the rm-core ``airm.kv_transports`` ``shm`` adapter
  engines     paged KV cache + block allocator, batched decode attention, the
              Llama decode step (LlamaDecoder) and prefill (LlamaPrefill)
  serving     continuous scheduling of decode streams onto the paged cache,
              prefetch, and the one-GPU prefill/decode run (pd_one_gpu)
"""
__version__ = "0.1.0"
