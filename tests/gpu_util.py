"""Moving oracle-format arrays to and from the GPU, and the tolerance rule of
the parity tests."""
from __future__ import annotations

import numpy as np
import torch

import oracle_lib as orc

TORCH_OF = {orc.F16: torch.float16, orc.BF16: torch.bfloat16, orc.F32: torch.float32}


def dev(arr: np.ndarray, code: int | None = None) -> torch.Tensor:
    """numpy bits -> cuda tensor of the matching dtype (bit-preserving)."""
    if code in (orc.F16, orc.BF16):
        return torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(TORCH_OF[code]).cuda()
    return torch.from_numpy(np.ascontiguousarray(arr)).cuda()


def host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def host_f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def half_ulp(ref: np.ndarray, code: int) -> np.ndarray:
    """Half a unit in the last place of the output dtype at |ref|: the
    rounding every correct kernel incurs when it stores its result."""
    mant = {orc.F16: 10, orc.BF16: 7, orc.F32: 23}[code]
    a = np.maximum(np.abs(ref), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(a)) - mant - 1)


def assert_close(got: torch.Tensor, ref: np.ndarray, code: int, atol: float, what: str = ""):
    """|got - ref| <= atol + half an output ulp at |ref| (ref is exact fp64)."""
    g = host_f64(got)
    assert g.shape == ref.shape, (g.shape, ref.shape)
    err = np.abs(g - ref)
    allowed = atol + half_ulp(ref, code)
    bad = ~(err <= allowed)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err - allowed, -np.inf)), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {err.size} outside tolerance; worst at {i}: "
                             f"got {g[i]!r} ref {ref[i]!r} err {err[i]:.3g} allowed {allowed[i]:.3g}; "
                             f"max err {err.max():.3g}")
