"""CPU oracle for the Qwen3-4B greedy decode path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may
import anything from this package, and only as the checker.  The product path
(``htn-2026_amd/``) never imports it: it runs the HIP library or raises.

Modules
  synth      deterministic counter-based generator of the synthetic checkpoint and prompts
             (numpy; bit-identical to the HIP generator ``qd_synth_bf16``), plus a minimal
             safetensors writer for an HF-format checkpoint directory.
  qwen3_ref  op-by-op torch-CPU restatement of transformers' Qwen3 forward
             (modeling_qwen3.py) with every bf16 rounding point of the reference
             (engine/kernels/rmsnorm.py:26-31, fused.py:65-74, fast.py:13-17), a greedy
             KV-cache loop (engine/engine.py:963-972), and the tree / chain verification
             forward (engine/kernels/tree.py, engine/spec.py).

How each oracle function is pinned is listed in the header of ``qwen3_ref``.
"""
