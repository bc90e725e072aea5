"""Parity bars shared by the GPU tests (test infrastructure).

Two bars, both must hold (written here):
  * absolute:     max |out - ref| <= ABS[dtype]                 2e-2 for bf16 inputs with fp32
                  accumulation, 1e-4 in the fp32-input validation mode;
  * scale-aware:  max |out - ref| <= REL[dtype] * max |ref|     2e-2 for bf16, 1e-3 for fp32.

The second bar is what discriminates at long key counts. With N(0,1) inputs the scores are ~N(0,1),
the softmax over ~45,000 keys is nearly flat and every output is a mean of ~45k values (|ref| ~ 0.03),
so the absolute bar alone passes a kernel that drops the last quarter of the keys or scales O by 1.5.
The reference's own check reports the reference's magnitude next to the error for the same reason
(`fwd_max_abs` beside `fwd_ref_max`, scripts/tests/test_pallas_attn.py:166-167).
`tests/test_parity_bars.py` shows on the CPU that both perturbations fail these bars at the C4 and
C3 key counts while the correctly rounded result passes.
"""
from __future__ import annotations

import numpy as np
import torch

ABS = {torch.bfloat16: 2e-2, torch.float32: 1e-4}
REL = {torch.bfloat16: 2e-2, torch.float32: 1e-3}


def _as_tensor(x, device) -> torch.Tensor:
    if isinstance(x, np.ndarray):
        return torch.from_numpy(x).to(device)
    return x.detach().to(device)


def errors(out, ref) -> tuple[float, float]:
    """(max |out - ref|, max |ref|) in float64, on out's device (CPU for numpy)."""
    device = out.device if torch.is_tensor(out) else torch.device("cpu")
    o = _as_tensor(out, device).double()
    r = _as_tensor(ref, device).double()
    if o.shape != r.shape:  # e.g. a [1, ...] slice against an unbatched reference
        r = r.reshape(o.shape) if r.numel() == o.numel() else torch.broadcast_tensors(o, r)[1]
    if o.numel() == 0:
        return 0.0, 0.0
    return float((o - r).abs().max()), float(r.abs().max())


def passes(out, ref, dtype, abs_tol=None, rel_tol=None) -> bool:
    err, scale = errors(out, ref)
    a = ABS[dtype] if abs_tol is None else abs_tol
    r = REL[dtype] if rel_tol is None else rel_tol
    return err <= a and err <= r * scale


def check(out, ref, dtype, what: str = "", abs_tol=None, rel_tol=None) -> float:
    """Assert both bars; returns the max abs error."""
    err, scale = errors(out, ref)
    a = ABS[dtype] if abs_tol is None else abs_tol
    r = REL[dtype] if rel_tol is None else rel_tol
    print(f"[parity] {what}: max abs err {err:.3e}, max |ref| {scale:.3e}", flush=True)
    assert err <= a, f"{what}: max abs err {err:.3e} > {a:.0e}"
    assert err <= r * scale, f"{what}: max abs err {err:.3e} > {r:.0e} x max|ref| {scale:.3e}"
    return err
