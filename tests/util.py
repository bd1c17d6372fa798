"""Error metrics shared by the parity tests."""

import torch


def normwise(got: torch.Tensor, ref: torch.Tensor) -> float:
    """max |got - ref| / max |ref| over all elements (0 when both are zero)."""
    got = got.detach().to("cpu", torch.float64)
    ref = ref.detach().to("cpu", torch.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if ref.numel() == 0:
        return 0.0
    scale = ref.abs().max().item()
    diff = (got - ref).abs().max().item()
    return diff / scale if scale > 0 else diff


def rel(got, ref) -> float:
    got, ref = float(got), float(ref)
    return abs(got - ref) / max(abs(ref), 1e-300)
