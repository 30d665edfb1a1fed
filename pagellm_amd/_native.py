"""ctypes binding of libpagellm_hip.so (C ABI in include/pagellm_hip.h).

The library is loaded from this package directory only; there is no
fallback of any kind: if it is missing or no GPU is present, every compute
call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().with_name("libpagellm_hip.so")

PLH_OK = 0
PLH_ERR_INVALID_ARG = -1
PLH_ERR_HIP = -2
PLH_ERR_OUT_OF_MEMORY = -3
PLH_ERR_UNSUPPORTED = -4
PLH_ERR_NO_DEVICE = -5
PLH_F32 = 0
PLH_F64 = 1
PLH_SAMPLE_ROWWISE = 1
PLH_SAMPLE_HIST_SPANS = 2
PLH_SAMPLE_NUCLEUS = 4
PLH_SAMPLE_NUCLEUS_ONLY = 8
PLH_OPT_KERNEL_TIMING = 1

_c_int, _c_i64, _c_sz, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/pagellm_hip.h
SIGNATURES = {
    "plh_abi_version": (_c_int, []),
    "plh_create": (_c_int, [ctypes.POINTER(_vp), _c_int]),
    "plh_destroy": (None, [_vp]),
    "plh_last_error": (ctypes.c_char_p, [_vp]),
    "plh_set_stream": (_c_int, [_vp, _vp]),
    "plh_set_option": (_c_int, [_vp, _c_int, _c_i64]),
    "plh_fallback_rows": (_c_int, [_vp, ctypes.POINTER(_c_i64)]),
    "plh_kernel_times": (_c_int, [_vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(_c_i64)]),
    "plh_alloc": (_c_int, [_vp, ctypes.POINTER(_vp), _c_sz]),
    "plh_free": (_c_int, [_vp, _vp]),
    "plh_h2d": (_c_int, [_vp, _vp, _vp, _c_sz]),
    "plh_d2h": (_c_int, [_vp, _vp, _vp, _c_sz]),
    "plh_host_alloc": (_c_int, [_vp, ctypes.POINTER(_vp), _c_sz]),
    "plh_host_free": (_c_int, [_vp, _vp]),
    "plh_h2d_async": (_c_int, [_vp, _vp, _vp, _c_sz]),
    "plh_sync": (_c_int, [_vp]),
    "plh_sample": (
        _c_int,
        [_vp, _vp, _c_int, _c_i64, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int],
    ),
    "plh_sample_noalloc": (
        _c_int,
        [_vp, _vp, _c_int, _c_i64, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int],
    ),
    "plh_penalize": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_int, _c_int, _vp, _vp, _vp, _vp, _c_i64]),
    "plh_draw": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_int, _c_int, _vp, _vp]),
    "plh_verify": (
        _c_int,
        [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _vp, _vp],
    ),
    "plh_append_ids": (_c_int, [_vp, _vp, _vp, _vp, _c_int]),
    "plh_copy_rows": (_c_int, [_vp, _vp, _c_i64, _vp, _c_i64, _c_i64, _c_int]),
    "plh_rmsnorm_lm_head": (
        _c_int,
        [_vp, _vp, _c_i64, _c_int, _c_int, _vp, ctypes.c_double, _vp, _c_i64, _c_int, _vp, _c_i64],
    ),
}

_lib = None
_lib_lock = threading.Lock()


def load_library() -> ctypes.CDLL:
    """Load (once) the in-tree shared library and declare its signatures."""
    global _lib
    with _lib_lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH.name} is not built; run `python -m pagellm_amd.build` "
                    "(the sampler has no CPU fallback)"
                )
            # One HIP runtime per process.  torch's ROCm wheel bundles its own
            # libamdhip64 (same soname as the system one); loaded first, it
            # also serves this library, so torch tensors and streams and this
            # library's calls share one runtime.  Loaded after the system
            # runtime, it would bring a second HIP/HSA runtime into the
            # process and torch would find no GPU.
            try:
                import torch  # noqa: F401
            except ImportError:
                pass
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


class PLHError(RuntimeError):
    """A HIP runtime failure reported by the library."""


def _raise(code: int, msg: str):
    if code == PLH_ERR_INVALID_ARG:
        raise ValueError(msg)
    if code == PLH_ERR_OUT_OF_MEMORY:
        raise MemoryError(msg)
    if code == PLH_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if code == PLH_ERR_NO_DEVICE:
        raise PLHError(f"no HIP device available: {msg}")
    raise PLHError(msg)


def _dtype_code(dt: np.dtype) -> int:
    if dt == np.float32:
        return PLH_F32
    if dt == np.float64:
        return PLH_F64
    raise TypeError(f"unsupported dtype {dt}; expected float32 or float64")


class DeviceArray:
    """A device allocation owned by a Context, with numpy-style metadata."""

    def __init__(self, ctx: "Context", shape, dtype):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        ptr = _vp()
        ctx._check(ctx.lib.plh_alloc(ctx.handle, ctypes.byref(ptr), max(self.nbytes, 1)))
        self.ptr = ptr.value

    def upload(self, host: np.ndarray) -> "DeviceArray":
        host = np.ascontiguousarray(host, dtype=self.dtype)
        if host.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: {host.nbytes} vs {self.nbytes}")
        self.ctx._check(self.ctx.lib.plh_h2d(self.ctx.handle, self.ptr, host.ctypes.data, host.nbytes))
        return self

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        self.ctx._check(self.ctx.lib.plh_d2h(self.ctx.handle, out.ctypes.data, self.ptr, self.nbytes))
        return out

    def free(self) -> None:
        if self.ptr and self.ctx.handle:
            self.ctx.lib.plh_free(self.ctx.handle, self.ptr)
        self.ptr = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One library context (device, stream, workspace).  Not thread-safe:
    use one per thread, as the reference samples from one engine thread."""

    def __init__(self, device: int | None = None):
        self.lib = load_library()
        if device is None:
            device = int(os.environ.get("PLH_DEVICE", "0"))
        h = _vp()
        rc = self.lib.plh_create(ctypes.byref(h), int(device))
        if rc != PLH_OK:
            _raise(rc, f"plh_create(device={device}) failed with code {rc}")
        self.handle = h.value
        self.device = device
        self._scratch: dict[str, DeviceArray] = {}
        self._pinned: dict[str, tuple[int, int]] = {}

    def _check(self, rc: int) -> None:
        if rc != PLH_OK:
            msg = self.lib.plh_last_error(self.handle)
            _raise(rc, msg.decode() if msg else f"error {rc}")

    def close(self) -> None:
        for buf in self._scratch.values():
            buf.free()
        self._scratch.clear()
        if self.handle:
            for ptr, _ in self._pinned.values():
                self.lib.plh_host_free(self.handle, ptr)
        self._pinned.clear()
        if self.handle:
            self.lib.plh_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------- buffers
    def empty(self, shape, dtype) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def to_device(self, host, dtype=None) -> DeviceArray:
        host = np.asarray(host) if dtype is None else np.asarray(host, dtype=dtype)
        return DeviceArray(self, host.shape, host.dtype).upload(host)

    def scratch(self, name: str, shape, dtype) -> DeviceArray:
        """A reusable device buffer, grown on demand (no allocation per call
        once warm)."""
        dtype = np.dtype(dtype)
        need = int(np.prod(shape, dtype=np.int64)) * dtype.itemsize
        buf = self._scratch.get(name)
        if buf is None or buf.nbytes < need:
            if buf is not None:
                buf.free()
            cap = max(need, 256)
            buf = DeviceArray(self, (cap,), np.uint8)
            self._scratch[name] = buf
        view = DeviceArray.__new__(DeviceArray)
        view.ctx, view.shape, view.dtype, view.nbytes, view.ptr = self, tuple(shape), dtype, need, buf.ptr
        view.free = lambda: None  # the cache owns the memory
        return view

    def scratch_upload(self, name: str, host) -> DeviceArray:
        host = np.ascontiguousarray(host)
        return self.scratch(name, host.shape, host.dtype).upload(host)

    def upload_rows(self, name: str, host: np.ndarray) -> tuple[DeviceArray, int]:
        """Upload [N, V] rows with the row stride padded to 16 bytes, so the
        sampling kernels take their 128-bit load path for any V (a 50 257-
        token vocabulary included).  Returns the buffer and the stride in
        elements; the pad columns are zero and never read."""
        host = np.asarray(host)
        n, v = host.shape
        es = host.dtype.itemsize
        ld = -(-v * es // 16) * 16 // es
        if ld != v:
            pad = np.empty((n, ld), host.dtype)
            pad[:, :v] = host
            pad[:, v:] = 0
            host = pad
        return self.scratch_upload(name, host), ld

    def pinned(self, name: str, nbytes: int) -> np.ndarray:
        """A reusable page-locked host buffer (uint8, at least nbytes), for
        plh_h2d_async; grown on demand."""
        buf = self._pinned.get(name)
        if buf is None or buf[1] < nbytes:
            if buf is not None:
                self._check(self.lib.plh_host_free(self.handle, buf[0]))
            cap = max(int(nbytes), 4096)
            ptr = _vp()
            self._check(self.lib.plh_host_alloc(self.handle, ctypes.byref(ptr), cap))
            buf = (ptr.value, cap)
            self._pinned[name] = buf
        return np.ctypeslib.as_array((ctypes.c_uint8 * buf[1]).from_address(buf[0]))

    def h2d_async(self, dst_ptr: int, src: np.ndarray) -> None:
        """Queue a copy of src (page-locked: from pinned()) to the device on
        the context's stream; src must stay unchanged until the stream has
        passed it (the next download or sync)."""
        self._check(self.lib.plh_h2d_async(self.handle, dst_ptr, src.ctypes.data, src.nbytes))

    def stage_upload(self, name: str, parts) -> list[int]:
        """Copy the host arrays in parts to one device buffer with a single
        queued copy from a page-locked host buffer, and return each array's
        device address (16-byte aligned).  Both buffers are reused by the
        next call with the same name, which the caller makes only after a
        download or sync has passed this copy."""
        arrs = [np.ascontiguousarray(a) for a in parts]
        offs, n = [], 0
        for a in arrs:
            offs.append(n)
            n += (a.nbytes + 15) & ~15
        d = self.scratch(name, (max(n, 16),), np.uint8)
        if n:
            stage = self.pinned(name, n)
            for a, o in zip(arrs, offs):
                stage[o:o + a.nbytes] = a.reshape(-1).view(np.uint8)
            self.h2d_async(d.ptr, stage[:n])
        return [d.ptr + o for o in offs]

    def sync(self) -> None:
        self._check(self.lib.plh_sync(self.handle))

    def set_stream(self, stream_handle: int | None) -> None:
        self._check(self.lib.plh_set_stream(self.handle, stream_handle or None))

    def fallback_rows(self) -> int:
        v = _c_i64()
        self._check(self.lib.plh_fallback_rows(self.handle, ctypes.byref(v)))
        return int(v.value)

    def set_kernel_timing(self, on: bool) -> None:
        self._check(self.lib.plh_set_option(self.handle, PLH_OPT_KERNEL_TIMING, 1 if on else 0))

    def kernel_times(self) -> tuple[float, float, int]:
        """(streaming-kernel ms, merge-kernel ms, calls) summed over the fast-path
        calls made since the last read while kernel timing was on."""
        a, b, n = ctypes.c_double(), ctypes.c_double(), _c_i64()
        self._check(self.lib.plh_kernel_times(self.handle, ctypes.byref(a), ctypes.byref(b), ctypes.byref(n)))
        return float(a.value), float(b.value), int(n.value)

    # ------------------------------------------------------------- kernels
    def sample(self, logits_ptr, dtype_code, ld, B, V, hist_ids, hist_off, temperature, top_k, top_p,
               rep_penalty, uniforms, out_ids, out_probs=None, flags=0) -> None:
        self._check(
            self.lib.plh_sample(
                self.handle, logits_ptr, dtype_code, ld, B, V, hist_ids, hist_off, temperature, top_k, top_p,
                rep_penalty, uniforms, out_ids, out_probs, flags,
            )
        )

    def sample_noalloc(self, logits_ptr, dtype_code, ld, B, V, hist_ids, hist_off, temperature, top_k, top_p,
                       rep_penalty, uniforms, out_ids, out_probs=None, flags=0) -> None:
        """plh_sample_noalloc: plh_sample with the fast path's workspace in the
        library's fixed per-GPU scratch array (no allocation during the call)."""
        self._check(
            self.lib.plh_sample_noalloc(
                self.handle, logits_ptr, dtype_code, ld, B, V, hist_ids, hist_off, temperature, top_k, top_p,
                rep_penalty, uniforms, out_ids, out_probs, flags,
            )
        )

    def penalize(self, x_ptr, dtype_code, ld, B, V, hist_ids, hist_off, rep_penalty, out_ptr, out_ld) -> None:
        self._check(
            self.lib.plh_penalize(self.handle, x_ptr, dtype_code, ld, B, V, hist_ids, hist_off, rep_penalty,
                                  out_ptr, out_ld)
        )

    def copy_rows(self, dst_ptr, dst_pitch, src_ptr, src_pitch, row_bytes, rows) -> None:
        self._check(self.lib.plh_copy_rows(self.handle, dst_ptr, int(dst_pitch), src_ptr, int(src_pitch),
                                           int(row_bytes), int(rows)))

    def rmsnorm_lm_head(self, h_ptr, ldh, N, D, norm_ptr, eps, w_ptr, ldw, V, out_ptr, ldo) -> None:
        self._check(self.lib.plh_rmsnorm_lm_head(self.handle, h_ptr, ldh, N, D, norm_ptr, eps, w_ptr, ldw, V,
                                                 out_ptr, ldo))

    def append_ids(self, slab_ptr, pos_ptr, ids_ptr, n) -> None:
        self._check(self.lib.plh_append_ids(self.handle, slab_ptr, pos_ptr, ids_ptr, int(n)))

    def draw(self, p_ptr, dtype_code, ld, B, V, uniforms, out_ids) -> None:
        self._check(self.lib.plh_draw(self.handle, p_ptr, dtype_code, ld, B, V, uniforms, out_ids))

    def verify(self, p_ptr, q_ptr, dtype_code, B, k, V, draft, accept_u, draw_u, per_stop, out_tokens,
               out_n_acc) -> None:
        self._check(
            self.lib.plh_verify(self.handle, p_ptr, q_ptr, dtype_code, B, k, V, draft, accept_u, draw_u,
                                int(per_stop), out_tokens, out_n_acc)
        )


_default: Context | None = None
_default_lock = threading.Lock()


def default_context() -> Context:
    """The process-wide context used by the drop-in functions."""
    global _default
    with _default_lock:
        if _default is None:
            _default = Context()
    return _default


def dtype_code(dt) -> int:
    return _dtype_code(np.dtype(dt))
