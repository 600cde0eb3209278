"""Helpers for the GPU parity tests: torch is used only for device memory and
the current stream; every computation goes through libcpi_hip.so."""
import ctypes

import numpy as np
import torch

from cpi_amd import _lib


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def dev(a: np.ndarray) -> torch.Tensor:
    """Upload a numpy array as raw bytes (uint8 device tensor, 16-B aligned)."""
    a = np.ascontiguousarray(a)
    t = torch.from_numpy(a.view(np.uint8).reshape(-1).copy()).cuda()
    return t


def empty(nbytes: int) -> torch.Tensor:
    return torch.zeros(max(nbytes, 16), dtype=torch.uint8, device="cuda")


_keep = []  # tensors whose raw pointers were handed out; freed at the next sync


def host(t: torch.Tensor, dtype, n=None) -> np.ndarray:
    torch.cuda.synchronize()
    _keep.clear()
    a = t.cpu().numpy().view(dtype)
    return a if n is None else a[:n]


def ptr(t) -> ctypes.c_void_p:
    if t is not None:
        _keep.append(t)
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def gemv(fmt: int, w, scales, scale_count, R, K, x, y, epilogue=_lib.EPI_STORE_F32, x_f32=True,
         norm_w=None, eps=1e-5, **kw):
    d = _lib.GemvDesc()
    _keep.extend(t for t in (w, scales, x, y, norm_w, *kw.values()) if isinstance(t, torch.Tensor))
    d.wfmt, d.w, d.scales, d.scale_count = fmt, w.data_ptr(), (scales.data_ptr() if scales is not None else 0), scale_count
    d.out_features, d.in_features = R, K
    d.x, d.x_is_f32 = x.data_ptr(), int(x_f32)
    d.norm_w = norm_w.data_ptr() if norm_w is not None else 0
    d.norm_eps = eps
    d.epilogue = epilogue
    d.y = y.data_ptr()
    for k, v in kw.items():
        setattr(d, k, v.data_ptr() if isinstance(v, torch.Tensor) else v)
    _lib.call("cpi_hip_gemv", ctypes.byref(d), stream())


def block_scales(s: np.ndarray, R: int, groups: int) -> np.ndarray:
    """Row-major fp16 group scales [R, groups] in the blocked layout of
    CPI_W_I4G32B: element ((r // 8) * groups + g) * 8 + r % 8, rows padded to a
    multiple of 8 with zeros."""
    rp = (R + 7) // 8 * 8
    a = np.zeros((rp, groups), np.float16)
    a[:R] = np.asarray(s, np.float16).reshape(R, groups)
    return np.ascontiguousarray(a.reshape(rp // 8, 8, groups).transpose(0, 2, 1)).reshape(-1)


def device_scales(fmt: str, s, R: int, K: int):
    """Scales as the device expects them for `fmt` (numpy, or None)."""
    if s is None:
        return None
    return block_scales(s, R, K // 32) if fmt == "i4g32b" else s
