"""Write tests/golden/moc_golden.npz: known-answer vectors of the MoC forward and
backward for the reference's own test matrix shape class (verify.py:16-18,
243-285: bf16/fp32 inputs, S in {2, 4}, plain / SiLU, fixed / varlen), at a size
the CPU oracle finishes in well under a second.

The reference ships no golden vectors; these are computed here, in fp64, by the
CPU oracle (oracle/moc_oracle.py), which tests/test_oracle.py pins against the
mathematics.  Inputs are drawn from seeded CPU generators and rounded to bf16
values, so that the same numbers feed the bf16 and the fp32 kernels exactly.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import moc_oracle as O  # noqa: E402

B, T, D, K = 2, 32, 32, 8
LENGTHS = [13, 1, 9, 5, 4]          # varlen: sum 32, a length-1 sequence included
OUT = Path(__file__).resolve().parent / "moc_golden.npz"


def cases():
    for varlen in (False, True):
        for S in (2, 4):
            for act in (None, "silu"):
                yield f"{'varlen' if varlen else 'fixed'}_S{S}_{act or 'none'}", varlen, S, act


def bf16_exact(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float64)


def make(seed: int, varlen: bool, S: int, act):
    g = torch.Generator().manual_seed(seed)
    lead = (sum(LENGTHS),) if varlen else (B, T)
    x = bf16_exact(0.5 * torch.randn(*lead, D, generator=g, dtype=torch.float64))
    alpha = bf16_exact(torch.softmax(torch.randn(*lead, K, generator=g, dtype=torch.float64), -1))
    basis = bf16_exact(0.1 * torch.randn(K, S, D, generator=g, dtype=torch.float64))
    dy = bf16_exact(0.1 * torch.randn(*lead, D, generator=g, dtype=torch.float64))
    if varlen:
        cu = torch.tensor([0] + list(np.cumsum(LENGTHS)), dtype=torch.int64)
        y, dx, da, db = O.moc_varlen_grads_ref(x, alpha, basis, cu, dy, act)
    else:
        cu = None
        y, dx, da, db = O.moc_grads_ref(x, alpha, basis, dy, act)
    out = {"x": x, "alpha": alpha, "basis": basis, "dy": dy, "y": y, "dx": dx, "dalpha": da,
           "dbasis": db}
    out = {k: v.numpy() for k, v in out.items()}
    if cu is not None:
        out["cu_seqlens"] = cu.numpy().astype(np.int32)
    return out


def main():
    arrays = {}
    for i, (name, varlen, S, act) in enumerate(cases()):
        for k, v in make(1000 + i, varlen, S, act).items():
            arrays[f"{name}/{k}"] = v.astype(np.float32) if v.dtype == np.float64 else v
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
