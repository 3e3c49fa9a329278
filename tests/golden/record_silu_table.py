"""Record bf16(silu(g)) for every bf16 bit pattern g, as the library's SwiGLU computes it.

The SwiGLU epilogues take silu of a bf16 value and round the result to bf16, so the function
is fully described by 65,536 outputs.  This table was written on MI355X by the library built
with the reference arithmetic of every SwiGLU path: torch's fp32 opmath x / (1 + exp(-x)) with
HIP's expf and an IEEE divide, then round-to-nearest-even to bf16.  tests/test_gpu_kernels.py
holds every later build to it bit for bit, so an evaluation of silu that is cheaper but has
to give the same bf16 results is checked over its whole domain.

Runs on the GPU (needs the built library):
    python tests/golden/record_silu_table.py [out.npy]      (default tests/golden/silu_bf16.npy)
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "htn-2026_amd"))


def silu_table(dev):
    """[65536] uint16: the library's bf16(silu(g)) for g = every bf16 bit pattern (qd_swiglu
    with the up half all 1.0, so bf16(bf16(silu(g)) * 1) = bf16(silu(g)))."""
    import torch

    from qdecode import ops
    pats = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    gu = torch.empty((1, 2 * 65536), dtype=torch.bfloat16, device=dev)
    gu[0, :65536] = pats.view(torch.bfloat16).to(dev)
    gu[0, 65536:] = 1.0
    out = ops.swiglu(gu)
    torch.cuda.synchronize()
    return out[0].cpu().view(torch.int16).numpy().astype("uint16")


def main():
    import numpy as np
    import torch
    path = sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(__file__), "silu_bf16.npy")
    tab = silu_table(torch.device("cuda:0"))
    np.save(path, tab)
    print(f"wrote {path}: {tab.shape[0]} entries")


if __name__ == "__main__":
    main()
