"""CPU: the local checkpoint reader (qdecode/checkpoint.py, the engine's counterpart of
``from_pretrained(model_path, local_files_only=True)``, reference engine/engine.py:237-247).

Checkpoints are written by oracle/synth.py at a small shape (the reader does not depend on the
model's dimensions) in the layouts an HF directory can take: one model.safetensors, or
several shards with a model.safetensors.index.json weight map; config.json with ``rope_theta``
or only a ``rope_parameters`` dict; tied or untied output projection.  Every tensor read back is
compared bit for bit with the generator's own bits (synth.param_bits), not with another read."""

import json
import os

import numpy as np
import pytest

from oracle import synth

SMALL = dict(synth.QWEN3_4B, hidden_size=256, intermediate_size=512, vocab_size=1000,
             num_attention_heads=8, num_key_value_heads=2)


@pytest.fixture(scope="module")
def ck():
    from qdecode import checkpoint
    return checkpoint


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("shards,rope_form,tied", [(1, "theta", True), (3, "parameters", True),
                                                   (2, "theta", False), (4, "parameters", False)])
def test_reader_returns_generator_bits(ck, tmp_path, shards, rope_form, tied):
    cfg = synth.write_checkpoint(str(tmp_path), seed=9, n_layers=2, cfg=SMALL, shards=shards,
                                 rope_form=rope_form, tied=tied)
    files = sorted(os.listdir(tmp_path))
    if shards > 1:
        assert "model.safetensors.index.json" in files
        assert sum(f.endswith(".safetensors") for f in files) == shards
    c = ck.read_config(str(tmp_path))
    assert c["rope_theta"] == 5000000.0
    assert c["tie_word_embeddings"] is tied
    assert (c["hidden_size"], c["num_key_value_heads"], c["head_dim"]) == (256, 2, 128)
    st = ck.SafeTensors(str(tmp_path))
    shapes = synth.param_shapes(cfg)
    assert set(st.entries) == set(shapes)
    assert ("lm_head.weight" in st) is (not tied)
    for name, shape in shapes.items():
        got = _bits(st.get(name))
        assert got.shape == tuple(shape), name
        assert np.array_equal(got, synth.param_bits(9, name, shape)), name
    if not tied:   # a real second matrix, not a copy of the embedding
        assert not np.array_equal(_bits(st.get("lm_head.weight")),
                                  _bits(st.get("model.embed_tokens.weight")))


def _config(tmp_path, **over):
    c = synth.hf_config(dict(SMALL, num_hidden_layers=1))
    c.update(over)
    for k in [k for k, v in over.items() if v is None]:
        del c[k]
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        json.dump(c, f)
    return str(tmp_path)


def test_config_defaults_follow_qwen3config(ck, tmp_path):
    """Absent keys take transformers' Qwen3Config defaults: untied head, theta 10000."""
    c = ck.read_config(_config(tmp_path, tie_word_embeddings=None, rope_theta=None))
    assert c["tie_word_embeddings"] is False
    assert c["rope_theta"] == 10000.0


@pytest.mark.parametrize("over", [
    {"rope_scaling": {"rope_type": "yarn", "factor": 4.0}},
    {"rope_scaling": {"type": "linear", "factor": 2.0}},
    {"rope_theta": None, "rope_parameters": {"rope_type": "dynamic", "rope_theta": 1e6}},
    {"use_sliding_window": True},
])
def test_config_rejects_what_the_kernels_do_not_compute(ck, tmp_path, over):
    with pytest.raises(ValueError):
        ck.read_config(_config(tmp_path, **over))


def test_config_accepts_default_scaling_entries(ck, tmp_path):
    c = ck.read_config(_config(tmp_path, rope_scaling={"rope_type": "default"},
                               use_sliding_window=False))
    assert c["rope_theta"] == 5000000.0


def test_missing_files_raise(ck, tmp_path):
    _config(tmp_path)
    with pytest.raises(FileNotFoundError):
        ck.SafeTensors(str(tmp_path))
