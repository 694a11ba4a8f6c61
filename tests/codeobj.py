"""Read the gfx950 code objects inside libkernelforge_hip.so (our own build).

The shared library's ``.hip_fatbin`` section holds one clang offload bundle
per translation unit. Each bundle is ``__CLANG_OFFLOAD_BUNDLE__`` followed by
an entry count and (offset, size, triple) records; the ``amdgcn`` entries are
ELF code objects. Kernel metadata comes from ``llvm-readelf --notes`` and the
instruction stream from ``llvm-objdump -d`` -- both on code this repository
compiled.
"""

from __future__ import annotations

import re
import struct
import subprocess
import tempfile
from dataclasses import dataclass, field
from functools import lru_cache
from pathlib import Path

LLVM = Path("/opt/rocm/llvm/bin")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


@dataclass
class KernelMeta:
    name: str
    vgprs: int = 0
    agprs: int = 0
    sgprs: int = 0
    private_bytes: int = 0
    group_bytes: int = 0
    asm: list[str] = field(default_factory=list)

    def count(self, mnemonic: str) -> int:
        """Instructions with this mnemonic, ignoring encoding suffixes (_e32, _e64, _dpp, _sdwa)."""
        return sum(1 for line in self.asm if _base(line.split(None, 1)[0]) == mnemonic)


_SUFFIXES = ("_e32", "_e64", "_dpp", "_sdwa")


def _base(op: str) -> str:
    for suffix in _SUFFIXES:
        if op.endswith(suffix):
            return op[: -len(suffix)]
    return op


def _fatbin(library: Path, workdir: Path) -> bytes:
    out = workdir / "fatbin.bin"
    subprocess.run(
        [str(LLVM / "llvm-objcopy"), f"--dump-section=.hip_fatbin={out}", str(library), str(workdir / "x.so")],
        check=True,
        capture_output=True,
    )
    return out.read_bytes()


def _code_objects(blob: bytes) -> list[bytes]:
    objs = []
    start = blob.find(MAGIC)
    while start >= 0:
        (count,) = struct.unpack_from("<Q", blob, start + len(MAGIC))
        pos = start + len(MAGIC) + 8
        for _ in range(count):
            offset, size, tlen = struct.unpack_from("<QQQ", blob, pos)
            triple = blob[pos + 24 : pos + 24 + tlen].decode()
            pos += 24 + tlen
            if triple.startswith("hip") and "gfx950" in triple and size:
                objs.append(blob[start + offset : start + offset + size])
        start = blob.find(MAGIC, start + len(MAGIC))
    return objs


def _parse_notes(text: str) -> dict[str, KernelMeta]:
    kernels: dict[str, KernelMeta] = {}
    for block in re.split(r"\n\s+- \.", text):
        name = re.search(r"\.name:\s+(\S+)", block)
        if not name or "group_segment_fixed_size" not in block:
            continue
        meta = KernelMeta(name=name.group(1))

        def grab(key: str) -> int:
            m = re.search(rf"\.{key}:\s+(\d+)", block)
            return int(m.group(1)) if m else 0

        meta.vgprs = grab("vgpr_count")
        meta.agprs = grab("agpr_count")
        meta.sgprs = grab("sgpr_count")
        meta.private_bytes = grab("private_segment_fixed_size")
        meta.group_bytes = grab("group_segment_fixed_size")
        kernels[meta.name] = meta
    return kernels


def _parse_asm(text: str, kernels: dict[str, KernelMeta]) -> None:
    current = None
    for line in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if m:
            current = kernels.get(m.group(1))
            continue
        if current is not None and line.startswith("\t"):
            current.asm.append(line.strip())


@lru_cache(maxsize=2)
def load_kernels(library: str) -> dict[str, KernelMeta]:
    """Every kernel in every gfx950 code object of ``library``, by mangled name."""
    kernels: dict[str, KernelMeta] = {}
    with tempfile.TemporaryDirectory() as tmp:
        work = Path(tmp)
        for i, co in enumerate(_code_objects(_fatbin(Path(library), work))):
            path = work / f"k{i}.co"
            path.write_bytes(co)
            notes = subprocess.run(
                [str(LLVM / "llvm-readelf"), "--notes", str(path)],
                check=True, capture_output=True, text=True,
            ).stdout
            found = _parse_notes(notes)
            asm = subprocess.run(
                [str(LLVM / "llvm-objdump"), "-d", "--mcpu=gfx950", str(path)],
                check=True, capture_output=True, text=True,
            ).stdout
            _parse_asm(asm, found)
            kernels.update(found)
    return kernels
