"""Shared helpers for the GPU parity tests: seeded inputs, host<->device moves
and the parity tolerance (2e-3 max-abs, 1e-3 relative, fp32 accumulation)."""
import numpy as np
import torch

from oracle import oracle as O

ATOL = 2e-3
RTOL = 1e-3


def dev(a: np.ndarray, device="cuda") -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).to(device).view(torch.uint32)
    return torch.from_numpy(a).to(device)


def host(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.uint32:
        return t.view(torch.int32).cpu().numpy().view(np.uint32)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def queries(rng, shape, dtype):
    """RMS-normed N(0,1) queries; returns (device tensor, exact float values)."""
    q32 = O.rms_norm(rng.standard_normal(shape).astype(np.float32))
    if dtype == "bf16":
        bits = O.f32_to_bf16_bits(q32)
        return (torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16),
                O.bf16_bits_to_f32(bits))
    if dtype == "f16":
        h = q32.astype(np.float16)
        return torch.from_numpy(h).cuda(), h.astype(np.float32)
    return torch.from_numpy(q32).cuda(), q32


def assert_close(got, ref, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    d = np.abs(got - ref)
    max_abs = float(d.max()) if d.size else 0.0
    rel = float(np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30)) if d.size else 0.0
    assert max_abs <= ATOL, f"{what}: max abs err {max_abs:.3e} > {ATOL}"
    assert rel <= RTOL, f"{what}: relative err {rel:.3e} > {RTOL}"
    return max_abs, rel
