"""The per-forward inputs of the block step (qd_block_step: prefill chunks, tree verification)
as one int64 block.  Kept apart from the runners so that host-only code (the tree loop and its
CPU tests) can build the pinned twin without loading the HIP library."""

import torch


class BlockInputs:
    """Every per-forward input of qd_block_step in ONE int64 block, so a host-side twin of the
    same layout (pinned) refreshes all of them with a single copy:

        tokens [B, T]   depth [B, T]   anc [B, T] (uint64 ancestor masks)   base [B]
        c_base [B]      c_src [B, T] int32          c_cnt [B] int32

    (the int32 fields take ceil(n / 2) words).  ``arrays()`` gives numpy views of a host block
    for writing rows in place."""

    FIELDS = (("tokens", 2, torch.int64), ("depth", 2, torch.int64), ("anc", 2, torch.int64),
              ("base", 1, torch.int64), ("c_base", 1, torch.int64), ("c_src", 2, torch.int32),
              ("c_cnt", 1, torch.int32))

    def __init__(self, B, T, device=None, pinned=False):
        self.B, self.T = B, T
        sizes = [B * T if rank == 2 else B for _, rank, _ in self.FIELDS]
        words = sum(n if dt == torch.int64 else (n + 1) // 2
                    for n, (_, _, dt) in zip(sizes, self.FIELDS))
        if pinned:
            self.block = torch.zeros((words,), dtype=torch.int64, pin_memory=True)
        else:
            self.block = torch.zeros((words,), dtype=torch.int64, device=device)
        off = 0
        for n, (name, rank, dt) in zip(sizes, self.FIELDS):
            w = n if dt == torch.int64 else (n + 1) // 2
            v = self.block[off:off + w]
            if dt != torch.int64:
                v = v.view(dt)[:n]
            setattr(self, name, v.view(B, T) if rank == 2 else v)
            off += w

    def arrays(self):
        """numpy views of the fields (host blocks only)."""
        return {name: getattr(self, name).numpy() for name, _, _ in self.FIELDS}
