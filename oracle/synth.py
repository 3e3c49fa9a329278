"""Deterministic synthetic Qwen3 checkpoint + prompts (CPU, numpy) -- test infrastructure.

The benchmark configs ask for "random-init bf16 N(0, 0.02) from seed s, norm weights = 1"
and prompts "uniform on [0, 151936)".  Both sides of every parity test (this CPU generator
and the device generator ``qd_synth_bf16`` in htn-2026_amd/csrc/synth.hip) must produce the
SAME bits, so the generator uses integer arithmetic plus exactly one IEEE fp32 multiply:

  key      = seed << 32 | stream              (stream = tensor id, see ``stream_id``)
  h_w(i)   = splitmix64 output number 2*i + w of the sequence seeded with ``key``
             (state_k = key + (k + 1) * 0x9E3779B97F4A7C15, finalised by mix64)
  S(i)     = sum of the eight 16-bit fields of h_0(i) and h_1(i)   (Irwin-Hall, n = 8)
  value(i) = bf16_rne( float32(S(i) - 262140) * float32(std / sigma_S) )

sigma_S = sqrt(8 * (65536^2 - 1) / 12) is the exact standard deviation of S, so the
values have mean 0 and standard deviation ``std`` (0.02); Irwin-Hall(8) is normal to within
0.3 % in its CDF and bounded at +-4.9 sigma.  Element i is the row-major index in the HF
[out_features, in_features] layout of the named tensor.

Prompt ids: uniform on [0, vocab) as mix64-hash modulo vocab (bias < 1e-14) on stream
``PROMPT_STREAM``.
"""

import json
import math
import os
import struct

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
SIGMA_S = math.sqrt(8.0 * (65536.0 ** 2 - 1.0) / 12.0)
S_MEAN = 4 * 65535                      # mean of the 8-term sum = 8 * 65535 / 2
PROMPT_STREAM = 0x7FFF0000
DRAFT_STREAM = 0x7FFE0000


def scale_for(std):
    """The fp32 multiplier applied to the centred integer sum (same value the device uses)."""
    return np.float32(std / SIGMA_S)


def stream_id(name):
    """Tensor id of an HF parameter name (the generator's stream)."""
    if name == "model.embed_tokens.weight":
        return 1
    if name == "lm_head.weight":                  # untied checkpoints only
        return 2
    parts = name.split(".")
    layer = int(parts[2])
    kind = {"q_proj": 0, "k_proj": 1, "v_proj": 2, "o_proj": 3,
            "gate_proj": 4, "up_proj": 5, "down_proj": 6}[parts[4]]
    return 16 + 16 * layer + kind


def _mix64(z):
    z = (z ^ (z >> np.uint64(30))) * M1
    z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def _hash_pair(seed, stream, idx):
    """(h_0(i), h_1(i)) for uint64 element indices ``idx``."""
    key = np.uint64((seed << 32) | stream)
    with np.errstate(over="ignore"):
        k0 = idx * np.uint64(2)
        h0 = _mix64(key + (k0 + np.uint64(1)) * GAMMA)
        h1 = _mix64(key + (k0 + np.uint64(2)) * GAMMA)
    return h0, h1


def _fields_sum(h):
    m = np.uint64(0xFFFF)
    return ((h & m) + ((h >> np.uint64(16)) & m) + ((h >> np.uint64(32)) & m)
            + (h >> np.uint64(48))).astype(np.int64)


def f32_to_bf16_bits(x):
    """Round-to-nearest-even fp32 -> bf16, returned as uint16 bit patterns (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounding = ((u >> np.uint32(16)) & np.uint32(1)) + np.uint32(0x7FFF)
    out = ((u + rounding) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    if nan.any():
        out[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return out


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16_bits(seed, stream, start, count, std=0.02):
    """bf16 bit patterns of elements [start, start + count) of one tensor stream."""
    idx = np.arange(start, start + count, dtype=np.uint64)
    h0, h1 = _hash_pair(seed, stream, idx)
    s = _fields_sum(h0) + _fields_sum(h1) - S_MEAN
    v = s.astype(np.float32) * scale_for(std)          # exactly one fp32 rounding
    return f32_to_bf16_bits(v)


_CLIB = None


def _clib():
    """The C restatement (oracle/csynth.c, built by oracle/Makefile) or None if not built."""
    global _CLIB
    if _CLIB is None:
        import ctypes
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build", "libcsynth.so")
        if not os.path.exists(path):
            return None
        lib = ctypes.CDLL(path)
        lib.oracle_synth_bf16.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64,
                                          ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float]
        lib.oracle_synth_bf16.restype = None
        _CLIB = lib
    return _CLIB


def normal_bf16_bits_c(seed, stream, start, count, std=0.02):
    """Same bits as ``normal_bf16_bits`` from the C restatement (OpenMP)."""
    lib = _clib()
    if lib is None:
        raise RuntimeError("oracle/_build/libcsynth.so is not built (make -C oracle)")
    out = np.empty(count, dtype=np.uint16)
    lib.oracle_synth_bf16(out.ctypes.data, seed, stream, start, count, float(scale_for(std)))
    return out


def tensor_bf16_bits(seed, name, shape, std=0.02, chunk=1 << 24):
    n = int(np.prod(shape))
    sid = stream_id(name)
    if _clib() is not None:
        return normal_bf16_bits_c(seed, sid, 0, n, std).reshape(shape)
    out = np.empty(n, dtype=np.uint16)
    for s in range(0, n, chunk):
        c = min(chunk, n - s)
        out[s:s + c] = normal_bf16_bits(seed, sid, s, c, std)
    return out.reshape(shape)


def prompt_ids(seed, batch, length, vocab=151936, stream=PROMPT_STREAM):
    idx = np.arange(batch * length, dtype=np.uint64)
    h0, _ = _hash_pair(seed, stream, idx)
    return (h0 % np.uint64(vocab)).astype(np.int64).reshape(batch, length)


# ------------------------------------------------------------------ model description
QWEN3_4B = dict(hidden_size=2560, intermediate_size=9728, num_attention_heads=32,
                num_key_value_heads=8, head_dim=128, vocab_size=151936, rms_norm_eps=1e-6,
                rope_theta=5000000.0, num_hidden_layers=36)


def param_shapes(cfg):
    H, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    nq = cfg["num_attention_heads"] * cfg["head_dim"]
    nkv = cfg["num_key_value_heads"] * cfg["head_dim"]
    D = cfg["head_dim"]
    shapes = {"model.embed_tokens.weight": (V, H), "model.norm.weight": (H,)}
    if not cfg.get("tie_word_embeddings", True):
        shapes["lm_head.weight"] = (V, H)
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        shapes.update({
            p + "input_layernorm.weight": (H,),
            p + "post_attention_layernorm.weight": (H,),
            p + "self_attn.q_proj.weight": (nq, H),
            p + "self_attn.k_proj.weight": (nkv, H),
            p + "self_attn.v_proj.weight": (nkv, H),
            p + "self_attn.o_proj.weight": (H, nq),
            p + "self_attn.q_norm.weight": (D,),
            p + "self_attn.k_norm.weight": (D,),
            p + "mlp.gate_proj.weight": (I, H),
            p + "mlp.up_proj.weight": (I, H),
            p + "mlp.down_proj.weight": (H, I),
        })
    return shapes


def param_bits(seed, name, shape, std=0.02):
    """One parameter as bf16 bits: norm weights are 1.0, everything else seeded N(0, std)."""
    if name.endswith("norm.weight"):
        return np.full(shape, 0x3F80, dtype=np.uint16)
    return tensor_bf16_bits(seed, name, shape, std)


def hf_config(cfg, rope_form="theta"):
    """config.json contents.  rope_form "theta" writes ``rope_theta`` (transformers 4.x form),
    "parameters" only a ``rope_parameters`` dict (the form transformers >= 5 writes)."""
    c = {
        "architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3",
        "hidden_size": cfg["hidden_size"], "intermediate_size": cfg["intermediate_size"],
        "num_hidden_layers": cfg["num_hidden_layers"],
        "num_attention_heads": cfg["num_attention_heads"],
        "num_key_value_heads": cfg["num_key_value_heads"], "head_dim": cfg["head_dim"],
        "vocab_size": cfg["vocab_size"], "rms_norm_eps": cfg["rms_norm_eps"],
        "tie_word_embeddings": bool(cfg.get("tie_word_embeddings", True)),
        "max_position_embeddings": 40960, "hidden_act": "silu", "attention_bias": False,
        "attention_dropout": 0.0, "torch_dtype": "bfloat16", "use_cache": True,
    }
    if rope_form == "theta":
        c["rope_theta"] = cfg["rope_theta"]
    elif rope_form == "parameters":
        c["rope_parameters"] = {"rope_type": "default", "rope_theta": cfg["rope_theta"]}
    else:
        raise ValueError(rope_form)
    return c


def _write_safetensors(path, names, shapes, seed, std, meta):
    header, off = {}, 0
    for n in names:
        nbytes = int(np.prod(shapes[n])) * 2
        header[n] = {"dtype": "BF16", "shape": list(shapes[n]), "data_offsets": [off, off + nbytes]}
        off += nbytes
    header["__metadata__"] = meta
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for n in names:
            f.write(param_bits(seed, n, shapes[n], std).tobytes())
    return off


def write_checkpoint(path, seed, n_layers, cfg=None, std=0.02, shards=1, rope_form="theta",
                     tied=True):
    """Write an HF checkpoint directory of the generator's weights: config.json plus
    model.safetensors (shards == 1) or model-0000i-of-0000n.safetensors files with a
    model.safetensors.index.json weight map (shards > 1, tensors dealt round-robin in name
    order so every file holds several kinds).  tied=False adds its own lm_head.weight
    (generator stream 2) and writes tie_word_embeddings false."""
    cfg = dict(cfg or QWEN3_4B)
    cfg["num_hidden_layers"] = n_layers
    cfg["tie_word_embeddings"] = bool(tied)
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(hf_config(cfg, rope_form), f, indent=1)
    shapes = param_shapes(cfg)
    names = sorted(shapes)
    meta = {"format": "pt", "generator": f"oracle.synth seed={seed} std={std}"}
    if shards <= 1:
        _write_safetensors(os.path.join(path, "model.safetensors"), names, shapes, seed, std, meta)
        return cfg
    files = [f"model-{i + 1:05d}-of-{shards:05d}.safetensors" for i in range(shards)]
    groups = [names[i::shards] for i in range(shards)]
    weight_map, total = {}, 0
    for fn, group in zip(files, groups):
        total += _write_safetensors(os.path.join(path, fn), group, shapes, seed, std, meta)
        weight_map.update({n: fn for n in group})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": total}, "weight_map": weight_map}, f, indent=1)
    return cfg
