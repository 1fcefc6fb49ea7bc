"""Shared helpers for the tests (device upload, tolerance checks)."""
import numpy as np

# Tolerance for fp16/fp32 outputs with fp32 accumulation, read as allclose:
# |got - ref| <= ATOL + RTOL * |ref|  (max-abs 1e-2, rel 1e-3).
ATOL = 1e-2
RTOL = 1e-3


def dev(arr, device):
    """numpy array -> torch tensor on `device` with the same bytes.
    uint32 -> int32, uint16 -> int16 storage (kernels see raw bits)."""
    import torch
    a = np.ascontiguousarray(arr)
    view = {np.dtype(np.uint32): np.int32, np.dtype(np.uint16): np.int16,
            np.dtype(np.uint8): np.uint8}.get(a.dtype)
    if view is not None:
        a = a.view(view)
    return torch.from_numpy(a).to(device)


def host_bits(t, dtype):
    """torch tensor -> numpy array reinterpreted as `dtype`."""
    import torch
    a = t.detach().cpu()
    if a.dtype in (torch.float16, torch.bfloat16):
        a = a.view(torch.int16)
    return a.numpy().view(dtype)


def to_f64(t):
    import torch
    return t.detach().to(torch.float64).cpu().numpy()


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    if bad.any():
        i = np.flatnonzero(bad.ravel())[:5]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} outside atol={atol} rtol={rtol}; "
            f"first at {i.tolist()}: got {got.ravel()[i].tolist()} ref {ref.ravel()[i].tolist()}; "
            f"max abs err {err.max():.3e}")


def inf_rel(got, ref):
    """The reference harness's metric: max|got-ref| / max|ref|
    (int4-gemv/src/main.mm:470-476)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(1e-30, np.max(np.abs(ref))))
