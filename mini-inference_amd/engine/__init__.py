"""MI355X-native paged KV-cache path: HIP kernels behind the reference engine's cache API.

Public modules:
  engine.kv_cache   PagedKVCache, PagedDecodeContext, PackedPrefillContext
  engine.model      Qwen2 harness (AttentionContext protocol, random-init decoder)
  engine.paged_ops  tensor-level kernel entry points (kv_append, paged_decode, copy_blocks)
  engine._native    ctypes binding of libmipaged.so (include/mipaged.h)
"""

__version__ = "0.1.0"
