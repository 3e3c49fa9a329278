"""MI355X-native Qwen3 greedy decode: host side of libqdecode.so.

  _lib        ctypes binding of the C ABI (include/qdecode.h); raises if the library is absent
  ops         tensor-level wrappers of each kernel (shape/dtype checks, stable buffers)
  checkpoint  local config.json + safetensors reader
  model       packed device weights, KV cache, decode / block runners, hipGraph capture
  tree        draft trees, greedy accept walk and the tree-verification stream
"""
