"""ctypes binding of ``libkernelforge_hip.so`` (declared in include/kernelforge_hip.h).

The library is loaded lazily on first use, never at import, so
``import kernelforge`` and every CPU-side module stay free of a HIP context
(the reference's import hygiene, tests/test_cpu_only_imports.py:22-84).

Status codes become exceptions whose class names drive the tuner's failure
classification (kernelforge/tuning/tuner.py:60-71): ``...OutOfResources`` and
``...Compil...`` are compile errors, ``...OutOfMemory...`` is an OOM, anything
else a runtime error. A missing library raises :class:`KernelLibraryNotCompiled`
-- there is no fallback path.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent.parent / "libkernelforge_hip.so"

KF_OK = 0
KF_ERR_INVALID_ARGUMENT = -1
KF_ERR_NOT_BUILT = -2
KF_ERR_OUT_OF_RESOURCES = -3
KF_ERR_LAUNCH = -4
KF_ERR_UNSUPPORTED_DTYPE = -5
KF_ERR_WORKSPACE = -6
KF_ERR_OUT_OF_MEMORY = -7

KF_EPILOGUE_NONE = 0
KF_EPILOGUE_BIAS_GELU = 1

KF_PIPELINE_STAGED = 0
KF_PIPELINE_DIRECT = 1

KF_WORKSPACE_COUNTERS = 1 << 18
KF_WORKSPACE_COUNTER_BYTES = 4 << 18
KF_GEMV_NO_ALLOC_SCRATCH_BYTES = 16 << 20


class KernelError(RuntimeError):
    """A status code other than KF_OK from the C-ABI."""

    code = 0


class KernelLibraryNotCompiled(KernelError):
    """libkernelforge_hip.so is absent or does not load."""


class KernelNotCompiled(KernelError):
    """The requested tile configuration has no ahead-of-time instantiation."""

    code = KF_ERR_NOT_BUILT


class KernelOutOfResources(KernelError):
    """The configuration exceeds LDS, register or workgroup limits."""

    code = KF_ERR_OUT_OF_RESOURCES


class KernelOutOfMemoryError(KernelError):
    code = KF_ERR_OUT_OF_MEMORY


class KernelInvalidArgument(KernelError):
    code = KF_ERR_INVALID_ARGUMENT


class KernelLaunchError(KernelError):
    code = KF_ERR_LAUNCH


class KernelWorkspaceError(KernelError):
    code = KF_ERR_WORKSPACE


_ERRORS: dict[int, type[KernelError]] = {
    KF_ERR_INVALID_ARGUMENT: KernelInvalidArgument,
    KF_ERR_NOT_BUILT: KernelNotCompiled,
    KF_ERR_OUT_OF_RESOURCES: KernelOutOfResources,
    KF_ERR_LAUNCH: KernelLaunchError,
    KF_ERR_UNSUPPORTED_DTYPE: KernelInvalidArgument,
    KF_ERR_WORKSPACE: KernelWorkspaceError,
    KF_ERR_OUT_OF_MEMORY: KernelOutOfMemoryError,
}

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

#: Exported symbol -> (restype, argtypes); mirrors include/kernelforge_hip.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "kf_abi_version": (_int, []),
    "kf_build_target": (ctypes.c_char_p, []),
    "kf_source_digest": (ctypes.c_char_p, []),
    "kf_last_error": (ctypes.c_char_p, []),
    "kf_stream_capture_id": (_int, [_vp, ctypes.POINTER(ctypes.c_ulonglong)]),
    "kf_gemm": (
        _int,
        [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int,
         _int, _int, _int, _int, _int, _int, _int, _vp],
    ),
    "kf_gemm_has_variant": (_int, [_int, _int, _int, _int, _int, _int, _int]),
    "kf_gemm_variant_count": (_int, []),
    "kf_gemm_variant_info": (
        _int,
        [_int] + [ctypes.POINTER(_int)] * 7,
    ),
    "kf_gemv": (
        _int,
        [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int,
         _int, _int, _int, _vp, _sz, _vp],
    ),
    "kf_gemv_workspace_bytes": (_sz, [_i64, _i64, _int]),
    "kf_gemv_no_alloc": (
        _int,
        [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int,
         _int, _int, _int, _vp],
    ),
    "kf_gemm_split_k": (
        _int,
        [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int,
         _int, _int, _int, _int, _int, _int, _int, _vp, _sz, _vp],
    ),
    "kf_gemm_workspace_bytes": (_sz, [_i64, _i64, _int, _int, _int]),
    "kf_gemm_concurrent_tiles": (_i64, [_int, _int, _int, _int, _int, _int, _int]),
    "kf_softmax": (_int, [_int, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, _int, _vp]),
    "kf_rmsnorm": (
        _int,
        [_int, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _int, _int, _int, _vp],
    ),
    "kf_rmsnorm_two_pass": (
        _int,
        [_int, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _int, _int, _int, _int,
         _vp],
    ),
    "kf_rmsnorm_two_pass_max_staged_cols": (_i64, [_int]),
    "kf_vector_add": (_int, [_int, _vp, _vp, _vp, _i64, _int, _int, _vp]),
}

#: kf_abi_version() of the library these signatures describe.
ABI_VERSION = 5

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load(path: str | Path | None = None) -> ctypes.CDLL:
    """Load the library once and bind every declared signature."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path is not None else LIBRARY_PATH
        if not target.exists():
            raise KernelLibraryNotCompiled(
                f"{target} is missing; build it with `python -m kernelforge.build` "
                "(or __graft_entry__.build())"
            )
        try:
            lib = ctypes.CDLL(str(target))
        except OSError as exc:
            raise KernelLibraryNotCompiled(f"cannot load {target}: {exc}") from exc
        version = lib.kf_abi_version()
        if version != ABI_VERSION:
            raise KernelLibraryNotCompiled(
                f"{target} has ABI version {version}, this package binds version {ABI_VERSION}; "
                "rebuild it with `python -m kernelforge.build`"
            )
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if path is None:
            _lib = lib
        return lib


def is_loaded() -> bool:
    return _lib is not None


def last_error() -> str:
    raw = load().kf_last_error()
    return raw.decode(errors="replace") if raw else ""


def source_digest() -> str:
    """The digest of the sources the loaded library was built from (``kf_source_digest``)."""
    return load().kf_source_digest().decode()


def check(rc: int, what: str) -> None:
    if rc == KF_OK:
        return
    cls = _ERRORS.get(rc, KernelError)
    raise cls(f"{what}: {last_error() or f'status {rc}'}")


def stream_of(tensor: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on the tensor's device."""
    return torch.cuda.current_stream(tensor.device).cuda_stream


def require_device_tensor(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError(
                f"expected a ROCm device tensor, got one on {t.device}; the HIP kernels have no "
                "CPU path"
            )
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"operands on different devices: {dev} vs {t.device}")


def gemm_variants() -> list[tuple[int, int, int, int, int, int, int]]:
    """(dtype code, BLOCK_M, BLOCK_N, BLOCK_K, waves, stages, pipeline) per compiled tile."""
    lib = load()
    out = []
    vals = [_int() for _ in range(7)]
    for i in range(lib.kf_gemm_variant_count()):
        check(lib.kf_gemm_variant_info(i, *[ctypes.byref(v) for v in vals]), "gemm variant info")
        out.append(tuple(v.value for v in vals))
    return out


def capture_id(stream: int) -> int:
    """Id of the graph capture ``stream`` is recording into, 0 when it is not capturing."""
    out = ctypes.c_ulonglong(0)
    check(load().kf_stream_capture_id(stream, ctypes.byref(out)), "stream capture query")
    return out.value


class _Workspaces:
    """Split-K workspaces: one per (device, stream) for eager calls, one per
    (device, stream, capture) for calls recorded into a HIP graph.

    Every split-K entry point (GEMV and GEMM) lays a workspace out the same
    way: a fixed region of arrival counters, then fp32 partial sums. The
    counters must be zero when a call starts and every completed call returns
    them to zero, so one buffer serves any sequence of calls in stream order.

    Eager buffers are cleared when made and replaced (the old one freed) when a
    call needs more; stream order makes both safe.

    A graph replays its kernels on the addresses it captured, long after the
    capture, and may be replayed on other streams. So a capture gets buffers of
    its own: created inside the capture (from the graph's memory pool), cleared
    by a fill node recorded at that point (so every replay starts from zero
    counters), shared only by later calls of the same capture, and never
    released: this object keeps a reference for the life of the process, so no
    later allocation can take memory a graph still writes. Two replays of one
    graph running at the same time share its buffers and race, like any
    concurrent use of one workspace.
    """

    def __init__(self) -> None:
        self._eager: dict[tuple[int, int], torch.Tensor] = {}
        self._captured: dict[tuple[int, int, int], torch.Tensor] = {}
        self._held: list[torch.Tensor] = []

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        dev = device.index if device.index is not None else torch.cuda.current_device()
        cap = capture_id(stream)
        if cap:
            key = (dev, stream, cap)
            buf = self._captured.get(key)
            if buf is None or buf.numel() < nbytes:
                buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
                self._captured[key] = buf
                self._held.append(buf)
            return buf
        key = (dev, stream)
        buf = self._eager.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self._eager[key] = buf
        return buf

    def held_for_graphs(self) -> int:
        """Bytes kept alive for captured graphs."""
        return sum(b.numel() for b in self._held)


workspaces = _Workspaces()
