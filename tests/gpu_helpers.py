"""Shared helpers of the GPU parity tests (tensor transfer and tolerances)."""
import numpy as np
import torch

# BASELINE.json tolerance for bf16 outputs: |gpu - ref| <= ATOL + RTOL * |ref|
RTOL = 1e-2
ATOL = 1e-3


def dev(a: np.ndarray, bf16: bool = False) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if bf16 or a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def bf(u16: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_bf16_close(got_u16, ref_u16, rtol=RTOL, atol=ATOL, what=""):
    g, r = bf(got_u16).astype(np.float64), bf(ref_u16).astype(np.float64)
    bad = np.abs(g - r) > atol + rtol * np.abs(r)
    if bad.any():
        i = np.flatnonzero(bad.reshape(-1))[:5]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} elements outside tolerance; first "
            f"{[(int(j), float(g.reshape(-1)[j]), float(r.reshape(-1)[j])) for j in i]}")


def assert_f32_close(got, ref, rtol=RTOL, atol=ATOL, what=""):
    g, r = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    bad = np.abs(g - r) > atol + rtol * np.abs(r)
    if bad.any():
        i = np.flatnonzero(bad.reshape(-1))[:5]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} outside tolerance; first "
            f"{[(int(j), float(g.reshape(-1)[j]), float(r.reshape(-1)[j])) for j in i]}")


def pack_ckpt(q: np.ndarray) -> np.ndarray:
    """int q in [-8, 7], [..., K] -> offset-binary bytes [..., K/2] (low nibble = even k)."""
    u = (q + 8).astype(np.uint8)
    return (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8)
