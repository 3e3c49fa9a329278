"""Local Hugging Face checkpoint reader: config.json + *.safetensors, no network, no transformers.

The reference loads the checkpoint with ``AutoModelForCausalLM.from_pretrained(model_path,
torch_dtype=bf16, local_files_only=True)`` (engine/engine.py:237-241) and takes the tied
lm_head from the embedding (engine.py:246-247).  This reader parses the safetensors header
itself (8-byte little-endian length + JSON), memory-maps each tensor and hands it to the caller
as a host torch tensor; single-file and sharded (model.safetensors.index.json) layouts are
both accepted.  A checkpoint without ``lm_head.weight`` (tie_word_embeddings) reuses the
embedding.
"""

import json
import os
import struct

import numpy as np
import torch

_DTYPES = {"BF16": (np.uint16, torch.bfloat16), "F16": (np.float16, torch.float16),
           "F32": (np.float32, torch.float32)}


def read_config(path):
    """Model dimensions from config.json, with transformers' Qwen3Config defaults for absent
    keys (rope_theta 10000, rms_norm_eps 1e-6, tie_word_embeddings False).  RoPE settings come
    from ``rope_theta`` or from a ``rope_parameters`` dict (transformers >= 5 writes this form);
    any RoPE scaling other than the default (``rope_scaling`` / ``rope_parameters.rope_type``:
    linear, dynamic, yarn, ...) is rejected, since the kernels implement plain RoPE."""
    with open(os.path.join(path, "config.json")) as f:
        c = json.load(f)
    rope = c.get("rope_parameters") or {}
    scaling = c.get("rope_scaling") or {}
    theta = c.get("rope_theta", rope.get("rope_theta", 10000.0))
    for src in (rope, scaling):
        kind = src.get("rope_type", src.get("type", "default"))
        if kind not in (None, "default"):
            raise ValueError(f"rope type {kind!r} is not supported (default RoPE only)")
    if c.get("use_sliding_window"):
        # Qwen3 then restricts layers >= max_window_layers to a key window; the kernels attend
        # over the whole cache
        raise ValueError("use_sliding_window is not supported (full attention only)")
    heads = c["num_attention_heads"]
    cfg = {
        "hidden_size": int(c["hidden_size"]),
        "intermediate_size": int(c["intermediate_size"]),
        "num_hidden_layers": int(c["num_hidden_layers"]),
        "num_attention_heads": int(heads),
        "num_key_value_heads": int(c.get("num_key_value_heads", heads)),
        "head_dim": int(c.get("head_dim") or c["hidden_size"] // heads),
        "vocab_size": int(c["vocab_size"]),
        "rms_norm_eps": float(c.get("rms_norm_eps", 1e-6)),
        "rope_theta": float(theta),
        "tie_word_embeddings": bool(c.get("tie_word_embeddings", False)),
    }
    return cfg


class SafeTensors:
    """Name -> memory-mapped tensor over every safetensors file of a checkpoint."""

    def __init__(self, path):
        self.path = path
        index = os.path.join(path, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                files = sorted(set(json.load(f)["weight_map"].values()))
        else:
            files = sorted(f for f in os.listdir(path) if f.endswith(".safetensors"))
        if not files:
            raise FileNotFoundError(f"no .safetensors files in {path}")
        self.entries = {}
        for fn in files:
            full = os.path.join(path, fn)
            with open(full, "rb") as f:
                (n,) = struct.unpack("<Q", f.read(8))
                header = json.loads(f.read(n))
            base = 8 + n
            for name, meta in header.items():
                if name == "__metadata__":
                    continue
                self.entries[name] = (full, meta["dtype"], tuple(meta["shape"]),
                                      base + meta["data_offsets"][0], base + meta["data_offsets"][1])

    def __contains__(self, name):
        return name in self.entries

    def get(self, name):
        """Host torch tensor (bf16/f16/f32 as stored), backed by a read-only memory map."""
        full, dt, shape, lo, hi = self.entries[name]
        if dt not in _DTYPES:
            raise TypeError(f"{name}: unsupported safetensors dtype {dt}")
        npdt, tdt = _DTYPES[dt]
        count = (hi - lo) // np.dtype(npdt).itemsize
        arr = np.memmap(full, dtype=npdt, mode="r", offset=lo, shape=(count,))
        t = torch.from_numpy(np.array(arr, copy=True))
        if tdt == torch.bfloat16:
            t = t.view(torch.int16).view(torch.bfloat16)
        return t.reshape(shape)
