"""Shared helpers for the GPU parity tests (host <-> device, error metrics)."""
import numpy as np
import torch


def to_dev(u16: np.ndarray, dev) -> torch.Tensor:
    """bf16 bit patterns (uint16) -> bf16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).view(torch.bfloat16).to(dev)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def f32_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy().astype(np.float32).view(np.uint32)


def maxabs_rel(got, ref) -> float:
    """max|got - ref| / max|ref| (the north-star's max-abs-normalised error)."""
    if isinstance(got, torch.Tensor):
        got = got.detach().float().cpu().numpy()
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-300))


def same_scales(got: np.ndarray, ref: np.ndarray) -> bool:
    """Bit equality of f32 scales, treating any NaN as equal to any NaN."""
    g = np.asarray(got, dtype=np.float32)
    r = np.asarray(ref, dtype=np.float32)
    both_nan = np.isnan(g) & np.isnan(r)
    return bool(np.all(both_nan | (g.view(np.uint32) == r.view(np.uint32))))


def as_dtype_values(v: np.ndarray, dt) -> np.ndarray:
    """f32 values rounded (RNE) to torch dtype dt's precision: what a tensor of dtype dt holds."""
    from oracle import bf16 as ob
    v = np.asarray(v, dtype=np.float32)
    if dt == torch.bfloat16:
        return ob.bf16_to_f32(ob.f32_to_bf16(v))
    if dt == torch.float16:
        return v.astype(np.float16).astype(np.float32)
    return v
