"""Device capabilities and provenance.

The search-space filters reason over a :class:`DeviceCaps` value object so they
can be tested on a machine without the GPU, as in the reference
(kernelforge/runtime/env.py:21-65). The fields are the ones gfx950 rules need:
CU count, LDS per workgroup, wave64, the 512-entry per-lane register file
(256 arch VGPRs + 256 AGPRs), XCD count, L2 and Infinity Cache (MALL) sizes,
and the peaks the roofline is priced against.

torch-ROCm reports some of these imprecisely (LDS opt-in, register count,
per-XCD L2), so known architectures are completed from a table keyed on
``gcnArchName``.
"""

from __future__ import annotations

import os
import platform
import socket
import sys
from dataclasses import asdict, dataclass, replace
from datetime import datetime, timezone

import torch


@dataclass(frozen=True)
class DeviceCaps:
    name: str
    gcn_arch: str
    total_memory_bytes: int
    cu_count: int
    lds_per_workgroup: int
    lds_per_cu: int
    vgprs_per_lane: int
    agprs_per_lane: int
    max_threads_per_workgroup: int
    wave_size: int
    xcd_count: int
    l2_cache_bytes: int
    mall_bytes: int
    peak_fp16_tflops: float
    peak_fp32_tflops: float
    peak_hbm_gbps: float
    #: False when the values were assumed rather than read from a device; any
    #: output derived from them must say so (env.py:31-36 in the reference).
    measured: bool = True

    # Reference-compatible aliases (the reference's filters say "SM").
    @property
    def sm_count(self) -> int:
        return self.cu_count

    @property
    def max_shared_memory_per_block(self) -> int:
        return self.lds_per_workgroup

    @property
    def warp_size(self) -> int:
        return self.wave_size

    @property
    def arch(self) -> str:
        return self.gcn_arch.split(":")[0]

    @property
    def key(self) -> str:
        """Cache key: full board name plus architecture, e.g. ``AMD_Instinct_MI355X_gfx950``.

        The board name is part of it for the reason the reference gives
        (env.py:49-65): two boards of one architecture can differ in CU count,
        cache and bandwidth, so a winner tuned on one is not assumed for the other.
        """
        safe = "".join(c if c.isalnum() else "_" for c in self.name).strip("_")
        while "__" in safe:
            safe = safe.replace("__", "_")
        return f"{safe}_{self.arch}"

    @property
    def flush_bytes(self) -> int:
        """Bytes a cache flush must overwrite: every L2 plus the Infinity Cache."""
        return self.l2_cache_bytes + self.mall_bytes


#: MI355X (gfx950) public specification. 256 CUs in 8 XCDs, 160 KiB LDS per
#: CU, 4 MiB L2 per XCD, 256 MiB Infinity Cache, 288 GB HBM3E at 8 TB/s,
#: dense fp16/bf16 MFMA 256 CU x 4096 FLOP/clk x 2.4 GHz = 2516.6 TFLOP/s.
MI355X_CAPS = DeviceCaps(
    name="AMD Instinct MI355X",
    gcn_arch="gfx950",
    total_memory_bytes=288 * 1000**3,
    cu_count=256,
    lds_per_workgroup=160 * 1024,
    lds_per_cu=160 * 1024,
    vgprs_per_lane=256,
    agprs_per_lane=256,
    max_threads_per_workgroup=1024,
    wave_size=64,
    xcd_count=8,
    l2_cache_bytes=8 * 4 * 1024 * 1024,
    mall_bytes=256 * 1024 * 1024,
    peak_fp16_tflops=2516.6,
    peak_fp32_tflops=157.3,
    peak_hbm_gbps=8000.0,
)

#: Fallback when no device is attached: the target, labelled as assumed.
_FALLBACK_CAPS = replace(MI355X_CAPS, name="AMD Instinct MI355X (assumed)", measured=False)

_ARCH_TABLE: dict[str, DeviceCaps] = {"gfx950": MI355X_CAPS}


def _device_available() -> bool:
    return torch.cuda.is_available() and torch.version.hip is not None


def device_caps(device: torch.device | str | int | None = None) -> DeviceCaps:
    """Capabilities of the attached device, or the assumed MI355X fallback."""
    if not _device_available():
        return _FALLBACK_CAPS
    index = 0 if device is None else (torch.device(device).index or 0)
    props = torch.cuda.get_device_properties(index)
    arch = str(getattr(props, "gcnArchName", "unknown"))
    base = _ARCH_TABLE.get(arch.split(":")[0])
    if base is None:
        # An architecture this build was not written for: keep what torch says.
        return DeviceCaps(
            name=props.name,
            gcn_arch=arch,
            total_memory_bytes=int(props.total_memory),
            cu_count=int(props.multi_processor_count),
            lds_per_workgroup=int(getattr(props, "shared_memory_per_block", 65536)),
            lds_per_cu=int(getattr(props, "shared_memory_per_multiprocessor", 65536)),
            vgprs_per_lane=256,
            agprs_per_lane=0,
            max_threads_per_workgroup=1024,
            wave_size=int(getattr(props, "warp_size", 64)),
            xcd_count=1,
            l2_cache_bytes=int(getattr(props, "L2_cache_size", 0)) or 4 * 1024 * 1024,
            mall_bytes=0,
            peak_fp16_tflops=0.0,
            peak_fp32_tflops=0.0,
            peak_hbm_gbps=0.0,
        )
    # Without libdrm's marketing-name table the runtime reports a generic
    # "AMD Radeon Graphics"; a known architecture with the table's CU count
    # is that board, and the cache key must not depend on the host's libdrm.
    name = props.name or base.name
    if "Instinct" not in name and int(props.multi_processor_count) == base.cu_count:
        name = base.name
    return replace(
        base,
        name=name,
        gcn_arch=arch,
        total_memory_bytes=int(props.total_memory),
        cu_count=int(props.multi_processor_count) or base.cu_count,
        measured=True,
    )


def device_key(device: torch.device | str | int | None = None) -> str:
    """Cache key for the attached device, or ``"cpu"`` when there is none.

    One derivation for both the recorded environment and the dispatch-time
    lookup (env.py:112-122): assumed caps must never name hardware that is
    not present.
    """
    if not _device_available():
        return "cpu"
    return device_caps(device).key


@dataclass(frozen=True)
class Environment:
    timestamp: str
    hostname: str
    platform: str
    python_version: str
    torch_version: str
    hip_version: str | None
    driver_version: str | None
    gpu_name: str | None
    gpu_arch: str | None
    gpu_memory_bytes: int | None
    cu_count: int | None
    device_key: str

    def as_dict(self) -> dict[str, object]:
        return asdict(self)

    def render(self) -> str:
        rows = [
            ("GPU", self.gpu_name or "none (CPU only)"),
            ("Architecture", self.gpu_arch or "-"),
            ("CU count", str(self.cu_count) if self.cu_count else "-"),
            (
                "VRAM",
                f"{self.gpu_memory_bytes / 1024**3:.1f} GiB" if self.gpu_memory_bytes else "-",
            ),
            ("HIP", self.hip_version or "-"),
            ("Driver", self.driver_version or "-"),
            ("PyTorch", self.torch_version),
            ("Python", self.python_version),
            ("Platform", self.platform),
            ("Host", self.hostname),
            ("Timestamp", self.timestamp),
        ]
        width = max(len(k) for k, _ in rows)
        return "\n".join(f"{k:<{width}}  {v}" for k, v in rows)


def _driver_version() -> str | None:
    try:
        with open("/sys/module/amdgpu/version") as handle:
            return handle.read().strip() or None
    except OSError:
        return None


def capture_environment(device: torch.device | str | int | None = None) -> Environment:
    has_gpu = _device_available()
    caps = device_caps(device) if has_gpu else None
    return Environment(
        timestamp=datetime.now(timezone.utc).isoformat(timespec="seconds"),
        hostname=socket.gethostname(),
        platform=platform.platform(),
        python_version=sys.version.split()[0],
        torch_version=torch.__version__,
        hip_version=torch.version.hip,
        driver_version=_driver_version() if has_gpu else None,
        gpu_name=caps.name if caps else None,
        gpu_arch=caps.gcn_arch if caps else None,
        gpu_memory_bytes=caps.total_memory_bytes if caps else None,
        cu_count=caps.cu_count if caps else None,
        device_key=device_key(device),
    )


def require_gpu() -> torch.device:
    """Fail loudly rather than silently measuring CPU latency (env.py:216-222)."""
    if not _device_available():
        raise RuntimeError(
            "kernelforge kernels require a ROCm GPU; torch.cuda.is_available() is False "
            f"(torch {torch.__version__}, HIP {torch.version.hip})."
        )
    return torch.device("cuda")


#: The reference's name for the same check.
require_cuda = require_gpu


def host_cores() -> int:
    """CPU threads available to this process (the CPU-baseline core count)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover - non-Linux
        return os.cpu_count() or 1
