"""Candidate generation, re-derived for gfx950.

The pipeline is the reference's (kernelforge/tuning/search.py:122-217):
enumerate a grid, reject each infeasible point with a *named* rule, drop
launches that cannot fill half the GPU (only when some candidate can), sort by
a documented priority and keep a budget. What changes is every number and
every rule: they come from the MI355X / CDNA4 machine model, not from an
NVIDIA SM.

Rules come in two kinds, kept apart as in the reference:

* **Instantiation rules** depend only on the tile and the dtype. They decide
  which configurations are compiled ahead of time (the build generates the
  HIP instantiation list from :func:`gemm_instantiations`), so a grid point
  they reject can never reach the device. These are hardware limits (LDS per
  workgroup, MFMA shapes, the per-lane register file) and one stated register
  budget heuristic.
* **Problem rules** depend on the shape (tile overshoot, split-K slices too
  short to fill a wave, rows per program beyond the row count).

Nothing here imports torch.cuda state beyond :class:`DeviceCaps`, so every rule
is unit-testable on a CPU-only host.
"""

from __future__ import annotations

import math
from abc import ABC, abstractmethod
from collections import Counter
from collections.abc import Iterator
from dataclasses import dataclass
from itertools import product

from kernelforge.dtypes import itemsize
from kernelforge.runtime.env import DeviceCaps, device_caps
from kernelforge.tuning.config import KernelConfig, Problem

#: Default candidate budget per problem (search.py:46 in the reference).
DEFAULT_MAX_CANDIDATES = 48

#: gfx950 MFMA output fragment: v_mfma_f32_16x16x32_{f16,bf16} and
#: v_mfma_f32_16x16x4_f32 all produce 16x16 fp32 tiles.
MFMA_TILE = 16


def mfma_fragment_edge(block_m: int, block_n: int, *, direct: int = 0, elem: int = 2) -> int:
    """Edge of the MFMA output fragments a tile is built from (gemm_direct.h DirectTile::MF).

    The direct pipeline's 256x256 tile multiplies with v_mfma_f32_32x32x16:
    its 64x128 wave tiles hold 128 accumulators per lane with either shape,
    but 32x32 fragments take half the fragment registers. Every other tile
    uses 16x16 fragments.
    """
    return 32 if direct and elem == 2 and block_m == 256 and block_n == 256 else MFMA_TILE

#: k consumed per MFMA step per fragment: 4 lane groups x 16 bytes of operand.
MFMA_K = {2: 32, 4: 16}

#: Hardware limit: bytes of one vector global load / LDS row pad.
VECTOR_BYTES = 16

#: Efficiency heuristic bounded by a hardware limit. A lane has 512 registers
#: (256 VGPR + 256 AGPR) at one wave per SIMD. fp32 accumulators above 128 per
#: lane leave too little room for the A/B fragments and the next slice's
#: staged global loads without spilling; 128 is a judgement, not a device
#: property (the compiled 256x128x64 / 4-wave tile uses 228 VGPR + 136 AGPR).
MAX_ACC_REGS_PER_LANE = 128

#: Registers (VGPR + AGPR) a SIMD holds per lane. A workgroup of W waves puts
#: ceil(W/4) waves on each SIMD, so each lane may use 512 / ceil(W/4).
REGISTER_FILE_PER_LANE = 512

#: Efficiency heuristic: of a lane's budget, this many are left for
#: addresses, loop state and the epilogue; the tile model (accumulators +
#: fragments + staged global loads) may claim the rest.
RESERVED_REGS_PER_LANE = 64


def register_budget(waves: int) -> int:
    """Registers one lane may use when a workgroup of ``waves`` waves is resident."""
    return REGISTER_FILE_PER_LANE // max(1, ceil_div(waves, 4))


def next_power_of_2(n: int) -> int:
    if n < 1:
        raise ValueError(f"expected a positive integer, got {n}")
    return 1 << (n - 1).bit_length()


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


@dataclass(frozen=True)
class CandidateSet:
    """What generation produced for one problem: the candidates in rank order,
    every rejected grid point with its rule, and the count after each stage."""

    problem: Problem
    generated: int
    feasible: int
    after_prune: int
    budget: int
    candidates: list[KernelConfig]
    rejected: tuple[tuple[KernelConfig, str], ...]

    def __len__(self) -> int:
        return len(self.candidates)

    def __iter__(self) -> Iterator[KernelConfig]:
        return iter(self.candidates)

    def rule_counts(self) -> list[tuple[str, int]]:
        """Rejections per rule name (the text before the first ``:`` or ``(``),
        most frequent first."""
        names = Counter(reason.split(":")[0].split("(")[0].strip() for _, reason in self.rejected)
        return sorted(names.items(), key=lambda kv: (-kv[1], kv[0]))


def _fill_prune(programs: dict[KernelConfig, int], cu_count: int) -> set[KernelConfig]:
    """Configs to drop because their launch fills under half the CUs.

    Applies only when some feasible config fills every CU: for a problem too
    small to fill the GPU at all, the small launches are the whole answer.
    """
    if not programs or max(programs.values()) < cu_count:
        return set()
    return {c for c, n in programs.items() if n < cu_count // 2}


class SearchSpace(ABC):
    """The configurations worth trying for one operation.

    Subclasses supply the grid, the named rejection rules, the launch size
    (for the fill prune) and the ranking key; :meth:`generate` runs the
    stages in a fixed order -- enumerate, reject, prune, rank, budget -- and
    keeps every count, which is what the published candidate counts pin.
    """

    operation: str

    def __init__(self, max_candidates: int = DEFAULT_MAX_CANDIDATES) -> None:
        if max_candidates < 1:
            raise ValueError(f"max_candidates must be positive, got {max_candidates}")
        self.max_candidates = max_candidates

    @abstractmethod
    def grid(self, problem: Problem) -> Iterator[KernelConfig]:
        """Every point of the unfiltered parameter grid."""

    @abstractmethod
    def reject_reason(self, config: KernelConfig, problem: Problem, caps: DeviceCaps) -> str | None:
        """The named rule that rules ``config`` out, or ``None`` to keep it."""

    def num_programs(self, config: KernelConfig, problem: Problem) -> int:
        """Workgroups the launch makes; spaces without a model skip the fill prune."""
        raise NotImplementedError

    def priority(self, config: KernelConfig, problem: Problem, caps: DeviceCaps) -> tuple[float, ...]:
        """Ranking key, lower first; ties break on the canonical JSON."""
        return (0.0,)

    def candidates(self, problem: Problem, caps: DeviceCaps | None = None, *,
                   max_candidates: int | None = None) -> list[KernelConfig]:
        return self.generate(problem, caps, max_candidates=max_candidates).candidates

    def generate(self, problem: Problem, caps: DeviceCaps | None = None, *,
                 max_candidates: int | None = None) -> CandidateSet:
        if problem.operation != self.operation:
            raise ValueError(
                f"{type(self).__name__} handles {self.operation!r}, got {problem.operation!r}")
        machine = caps or device_caps()
        budget = self.max_candidates if max_candidates is None else max_candidates
        if budget < 1:
            raise ValueError(f"max_candidates must be positive, got {budget}")

        points = list(self.grid(problem))
        verdicts = [(c, self.reject_reason(c, problem, machine)) for c in points]
        rejected = [(c, why) for c, why in verdicts if why is not None]
        feasible = [c for c, why in verdicts if why is None]

        try:
            programs = {c: self.num_programs(c, problem) for c in feasible}
        except NotImplementedError:
            programs = {}
        dropped = _fill_prune(programs, machine.cu_count)
        rejected += [(c, f"underfilled: launch grid of {programs[c]} workgroups fills under half "
                         f"of {machine.cu_count} CUs") for c in feasible if c in dropped]
        survivors = [c for c in feasible if c not in dropped]
        ranked = sorted(survivors, key=lambda c: (*self.priority(c, problem, machine), c.to_json()))
        return CandidateSet(problem=problem, generated=len(points), feasible=len(feasible),
                            after_prune=len(ranked), budget=budget,
                            candidates=self.select(ranked, budget, problem),
                            rejected=tuple(rejected))

    def select(self, ranked: list[KernelConfig], budget: int, problem: Problem) -> list[KernelConfig]:
        """The candidates the budget measures, from the ranked survivors."""
        return ranked[:budget]

    def explain(self, problem: Problem, caps: DeviceCaps | None = None) -> str:
        """The stage counts and rejections by rule, for ``tune --explain``."""
        machine = caps or device_caps()
        out = self.generate(problem, machine)
        note = "" if machine.measured else "  <- no device attached"
        lines = [
            problem.describe(),
            f"  device           : {machine.name} ({machine.arch}), {machine.cu_count} CUs, "
            f"{machine.lds_per_workgroup // 1024} KiB LDS/workgroup, wave{machine.wave_size}{note}",
            f"  grid points      : {out.generated}",
            f"  feasible         : {out.feasible}",
            f"  after prune      : {out.after_prune}",
            f"  selected (budget): {len(out.candidates)} of {out.budget}",
        ]
        counts = out.rule_counts()
        if counts:
            lines.append("  rejections by rule:")
            lines += [f"    {n:>4}  {rule}" for rule, n in counts]
        return "\n".join(lines)


# ---------------------------------------------------------------------------
# GEMM (matmul, fused_linear): MFMA tiles, plus split-K GEMV for decode rows.
# ---------------------------------------------------------------------------


def wave_grid(waves: int, block_m: int, block_n: int) -> tuple[int, int]:
    """How the kernel arranges its waves over the tile (gemm_impl.h WaveGrid)."""
    if waves == 4:
        return 2, 2
    if waves == 8:
        return (4, 2) if block_m >= block_n else (2, 4)
    return 1, waves


def gemm_lds_bytes(block_m: int, block_n: int, block_k: int, stages: int, elem: int) -> int:
    """LDS of the double-buffered A/B stages, k-contiguous rows padded by 16 bytes."""
    pad = VECTOR_BYTES // elem
    return stages * (block_m + block_n) * (block_k + pad) * elem


def gemm_tile_regs(
    block_m: int, block_n: int, block_k: int, waves: int, elem: int, *, direct: int = 0
) -> dict[str, int]:
    """Per-lane register model of one tile: accumulators, fragments, staged loads.

    The direct pipeline stages nothing in registers (the DMA writes LDS) but
    holds two k steps of fragments: the second step's are read while the
    first step's MFMAs run.
    """
    lanes = waves * 64
    wm, wn = wave_grid(waves, block_m, block_n)
    acc = block_m * block_n // lanes
    edge = mfma_fragment_edge(block_m, block_n, direct=direct, elem=elem)
    frags = 4 * (block_m // wm // edge + block_n // wn // edge) * (2 if direct else 1)
    staged = 0 if direct else 4 * ceil_div((block_m + block_n) * block_k * elem, VECTOR_BYTES * lanes)
    return {"acc": acc, "frags": frags, "staged": staged, "total": acc + frags + staged}


#: The direct-to-LDS pipeline moves one 128-byte row segment of each operand
#: row per k-slice.
DIRECT_ROW_BYTES = 128
#: Its BLOCK_K for 16-bit inputs (fp32: direct_block_k(4) = 32).
DIRECT_BLOCK_K = DIRECT_ROW_BYTES // 2


def direct_block_k(elem: int) -> int:
    """Elements of a direct k-slice: one 128-byte row segment."""
    return DIRECT_ROW_BYTES // elem


def gemm_direct_lds_bytes(block_m: int, block_n: int, stages: int) -> int:
    """LDS of the direct pipeline: dense (unpadded, swizzled) stages of 128-byte rows."""
    return stages * (block_m + block_n) * DIRECT_ROW_BYTES


def gemm_direct_static_lds_bytes(block_m: int, block_n: int, stages: int) -> int:
    """The direct kernel's static LDS (gemm_direct.h DirectTile::kLdsBytes).

    The stages, except on the 32x32x16 path, whose staged C tile (rows of
    BLOCK_N + 8 16-bit elements) is larger than its two stages and sets the size.
    """
    lds = gemm_direct_lds_bytes(block_m, block_n, stages)
    if mfma_fragment_edge(block_m, block_n, direct=1) == 32:
        lds = max(lds, block_m * (block_n + 8) * 2)
    return lds


def gemm_direct_reason(
    block_m: int, block_n: int, block_k: int, waves: int, stages: int, elem: int, caps: DeviceCaps
) -> str | None:
    """Extra shape-independent rules of the direct (global->LDS DMA) pipeline."""
    if block_k != direct_block_k(elem):
        return (f"direct DMA: BLOCK_K must be {direct_block_k(elem)} for {elem}-byte inputs "
                "(one 128-byte row segment per slice)")
    if elem == 4 and block_m == 256 and block_n == 256:
        return "direct DMA: the 256x256 tile multiplies with 16-bit 32x32x16 MFMAs only"
    lanes = waves * 64
    if elem == 4 and block_m * block_n // lanes > 64:
        # Measured: the 4-wave 128x256 and 256x128 fp32 tiles spill 8-160 bytes
        # per lane (a B fragment is four 4-byte reads, each its own address).
        return (f"direct DMA: {block_m * block_n // lanes} fp32 accumulators per lane leave no "
                "registers for the fp32 fragment reads")
    chunks = DIRECT_ROW_BYTES // VECTOR_BYTES  # 16-byte chunks per row
    if (block_m * chunks) % lanes or (block_n * chunks) % lanes:
        return f"direct DMA: {block_m}x{block_n} slices do not split into whole 16-byte chunks per lane"
    if block_n < 64:
        return f"direct DMA: BLOCK_N={block_n} leaves too few chunks per row for the bank swizzle"
    lds = gemm_direct_lds_bytes(block_m, block_n, stages)
    if lds > caps.lds_per_workgroup:
        return (
            f"LDS: {lds // 1024} KiB of A/B stages exceeds the "
            f"{caps.lds_per_workgroup // 1024} KiB per-workgroup limit"
        )
    return None


def gemm_instantiation_reason(
    block_m: int,
    block_n: int,
    block_k: int,
    waves: int,
    stages: int,
    elem: int,
    caps: DeviceCaps,
    direct: int = 0,
) -> str | None:
    """Shape-independent rules: why this tile is not compiled, or ``None``."""
    if direct:
        reason = gemm_direct_reason(block_m, block_n, block_k, waves, stages, elem, caps)
        if reason is not None:
            return reason
    elif stages != 2:
        return f"pipeline: the register-staged pipeline is double-buffered, not {stages}-stage"
    kstep = MFMA_K[elem]
    if block_k % kstep:
        return f"MFMA k step: BLOCK_K={block_k} is not a multiple of {kstep} for {elem}-byte inputs"
    wm, wn = wave_grid(waves, block_m, block_n)
    if block_m % (MFMA_TILE * wm) or block_n % (MFMA_TILE * wn):
        return (
            f"wave tile: {block_m}x{block_n} over {wm}x{wn} waves is not whole "
            f"{MFMA_TILE}x{MFMA_TILE} MFMA fragments"
        )
    lds = gemm_lds_bytes(block_m, block_n, block_k, stages, elem)
    if not direct and lds > caps.lds_per_workgroup:
        return (
            f"LDS: {lds // 1024} KiB of A/B stages exceeds the "
            f"{caps.lds_per_workgroup // 1024} KiB per-workgroup limit"
        )
    regs = gemm_tile_regs(block_m, block_n, block_k, waves, elem, direct=direct)
    if regs["acc"] > MAX_ACC_REGS_PER_LANE:
        return f"register pressure: {regs['acc']} accumulator registers per lane"
    budget = register_budget(waves) - RESERVED_REGS_PER_LANE
    if regs["total"] > budget:
        return (
            f"register file: {regs['total']} tile registers per lane exceed the "
            f"{budget} available at {waves} waves"
        )
    return None


#: Lanes per row segment of a GEMV config that does not name it (the strip
#: width of the first GEMV, kept so that older cached configs keep their meaning).
GEMV_DEFAULT_LANES_PER_ROW = 64


def gemv_unroll(rows: int) -> int:
    """Rows of W each lane loads per trip (gemv.hip gemv_unroll); trips are
    double buffered, so twice as many are in flight."""
    return 8 if rows <= 1 else (4 if rows <= 2 else 2)


class _GemmSpace(SearchSpace):
    """Shared by matmul and fused_linear: same main loop, different epilogue."""

    BLOCK_M = (32, 64, 128, 256)
    BLOCK_N = (32, 64, 128, 256)
    BLOCK_K = (16, 32, 64)
    NUM_WARPS = (4, 8)
    #: LDS stages: the register-staged pipeline is double-buffered; the DMA
    #: pipeline can keep two slices in flight with a third stage.
    NUM_STAGES = (2, 3)
    #: 0: register-staged LDS pipeline; 1: global->LDS DMA pipeline.
    DIRECT = (0, 1)
    #: Rows of tiles per launch-order band: derived from the tile by
    #: :func:`gemm_group_m` rather than searched (it changes traffic, not time).

    #: Split-K GEMV grid, offered when M is at most GEMV_MAX_M.
    GEMV_MAX_M = 8
    SPLIT_K = (1, 2, 4, 8, 16, 32, 64)
    GEMV_WARPS = (1, 2, 4, 8, 16)
    #: Lanes per row segment: a strip is LANES_PER_ROW 16-byte vectors wide and
    #: one wave load covers 64 / LANES_PER_ROW rows.
    GEMV_LANES_PER_ROW = (8, 16, 32, 64)
    #: Dynamic LDS the GEMV wave reduction may use (gemv.hip kGemvMaxLds).
    GEMV_MAX_LDS = 64 * 1024
    #: Split-K for DMA tiles: programs per output tile, offered while the
    #: unsplit tiles leave CUs idle (few rows: prefill of short prompts,
    #: batched decode).
    TILE_SPLIT_K = (2, 4, 8, 16)
    #: Fewest k-slices (of 64) a split program may own: below this the
    #: pipeline's fill and the partial-tile traffic dominate.
    TILE_SPLIT_MIN_SLICES = 4

    def grid(self, problem: Problem) -> Iterator[KernelConfig]:
        for direct, bm, bn, bk, warps, stages in product(
            self.DIRECT, self.BLOCK_M, self.BLOCK_N, self.BLOCK_K, self.NUM_WARPS, self.NUM_STAGES
        ):
            yield KernelConfig(
                self.operation,
                BLOCK_M=bm,
                BLOCK_N=bn,
                BLOCK_K=bk,
                GROUP_M=gemm_group_m(bm, bn),
                DIRECT=direct,
                num_warps=warps,
                num_stages=stages,
            )
        for bm, bn, warps, stages, split in product(
            self.BLOCK_M, self.BLOCK_N, self.NUM_WARPS, self.NUM_STAGES, self.TILE_SPLIT_K
        ):
            yield KernelConfig(
                self.operation,
                BLOCK_M=bm,
                BLOCK_N=bn,
                BLOCK_K=direct_block_k(itemsize(problem.dtype)),
                GROUP_M=gemm_group_m(bm, bn),
                DIRECT=1,
                SPLIT_K=split,
                num_warps=warps,
                num_stages=stages,
            )
        if problem.dims_dict["M"] <= self.GEMV_MAX_M:
            for split, lanes, warps in product(self.SPLIT_K, self.GEMV_LANES_PER_ROW, self.GEMV_WARPS):
                yield KernelConfig(
                    self.operation, GEMV=1, SPLIT_K=split, LANES_PER_ROW=lanes, num_warps=warps
                )

    #: Decode batches of at least this many rows keep a third of the budget for
    #: MFMA tiles, which rank behind every GEMV candidate: at 8 rows a split
    #: 32-row tile can beat the strip kernel, whose per-lane accumulators grow
    #: with the rows.
    GEMV_SHARED_BUDGET_M = 4

    def select(self, ranked: list[KernelConfig], budget: int, problem: Problem) -> list[KernelConfig]:
        m = problem.dims_dict["M"]
        if not self.GEMV_SHARED_BUDGET_M <= m <= self.GEMV_MAX_M:
            return ranked[:budget]
        gemv = [c for c in ranked if c.get("GEMV")]
        tiles = [c for c in ranked if not c.get("GEMV")]
        keep = gemv[: budget - min(len(tiles), budget // 3)]
        return keep + tiles[: budget - len(keep)]

    def num_programs(self, config: KernelConfig, problem: Problem) -> int:
        dims = problem.dims_dict
        if config.get("GEMV"):
            lanes = config.get("LANES_PER_ROW", GEMV_DEFAULT_LANES_PER_ROW)
            if problem.layout == "bt":
                # gemv_dot: a wave load covers 64/lanes columns, a block num_warps of those.
                return ceil_div(dims["N"], config["num_warps"] * (64 // lanes)) * config["SPLIT_K"]
            strip = lanes * (VECTOR_BYTES // problem.itemsize)
            return ceil_div(dims["N"], strip) * config["SPLIT_K"]
        tiles = ceil_div(dims["M"], config["BLOCK_M"]) * ceil_div(dims["N"], config["BLOCK_N"])
        return tiles * config.get("SPLIT_K", 1)

    def reject_reason(self, config: KernelConfig, problem: Problem, caps: DeviceCaps) -> str | None:
        dims = problem.dims_dict
        m, n, k = dims["M"], dims["N"], dims["K"]
        elem = itemsize(problem.dtype)
        if config.get("GEMV"):
            if problem.layout == "bt":
                return self._gemv_dot_reason(config, m, k, elem)
            return self._gemv_reason(config, m, k, elem)

        bm, bn = config["BLOCK_M"], config["BLOCK_N"]
        reason = gemm_instantiation_reason(
            bm,
            bn,
            config["BLOCK_K"],
            config["num_warps"],
            config["num_stages"],
            elem,
            caps,
            direct=config.get("DIRECT", 0),
        )
        if reason is not None:
            return reason
        # A tile more than twice the problem computes thrown-away work. As in
        # the reference (search.py:370-386), the rule yields while no smaller
        # tile exists in the grid, so tiny problems keep a candidate.
        if bm > 2 * m and bm > min(self.BLOCK_M):
            return f"tile overshoot: BLOCK_M={bm} for M={m}"
        if bn > 2 * n and bn > min(self.BLOCK_N):
            return f"tile overshoot: BLOCK_N={bn} for N={n}"
        split = config.get("SPLIT_K", 1)
        if split > 1:
            if not config.get("DIRECT"):
                return "split-K tiles: only the DMA pipeline splits K"
            tiles = ceil_div(m, bm) * ceil_div(n, bn)
            round_ = caps.cu_count * gemm_resident_workgroups(config, caps)
            # Only the tiles of the last, partial round are split (all of them
            # when there is a single round); the kernel runs the rest unsplit.
            tail = tiles % round_ if tiles >= round_ else tiles
            if tail == 0:
                return f"split-K tiles: {tiles} tiles fill whole rounds of {round_} workgroups"
            if tail * split > round_:
                # Measured: a second round of split programs costs more than
                # the split saves (512x11008x4096: 256x128 at 65 us unsplit,
                # 87 us at SPLIT_K=2, 108 us at 4; 2048x11008x4096: 197 us
                # unsplit, 215 us when its 176-tile last round is split in two).
                return (
                    f"split-K tiles: {tail} split tiles x {split} exceed one round of "
                    f"{round_} workgroups"
                )
            slices = ceil_div(ceil_div(k, 64), split)
            if slices < self.TILE_SPLIT_MIN_SLICES:
                return (
                    f"split-K slice too short: {slices} k-slices per program at SPLIT_K={split} "
                    f"(fewest {self.TILE_SPLIT_MIN_SLICES})"
                )
        return None

    def _gemv_reason(self, config: KernelConfig, m: int, k: int, elem: int) -> str | None:
        warps, split = config["num_warps"], config["SPLIT_K"]
        lanes = config.get("LANES_PER_ROW", GEMV_DEFAULT_LANES_PER_ROW)
        mr = next_power_of_2(m)
        max_warps = 16 if mr == 4 else 8
        if warps > max_warps:
            return f"register pressure: {mr} rows of x allow at most {max_warps} waves, got {warps}"
        lds = warps * mr * lanes * (VECTOR_BYTES // elem) * 4
        if lds > self.GEMV_MAX_LDS:
            return f"LDS: wave reduction needs {lds // 1024} KiB at num_warps={warps}, M={m}"
        slice_rows = ceil_div(k, split)
        in_flight = warps * (64 // lanes) * gemv_unroll(mr)
        if split > 1 and slice_rows < in_flight:
            return (
                f"split-K slice too short: {slice_rows} rows of K for {warps} waves x "
                f"{64 // lanes} rows x {gemv_unroll(mr)} in flight"
            )
        return None

    def _gemv_dot_reason(self, config: KernelConfig, m: int, k: int, elem: int) -> str | None:
        """gemv_dot (k-contiguous W): lanes split one column's k-run into 16-byte
        vectors, so a slice needs at least one vector per lane."""
        warps, split = config["num_warps"], config["SPLIT_K"]
        lanes = config.get("LANES_PER_ROW", GEMV_DEFAULT_LANES_PER_ROW)
        mr = next_power_of_2(m)
        max_warps = 16 if mr == 4 else 8
        if warps > max_warps:
            return f"register pressure: {mr} rows of x allow at most {max_warps} waves, got {warps}"
        slice_k = ceil_div(k, split)
        if split > 1 and slice_k < lanes * (VECTOR_BYTES // elem):
            return f"split-K slice too short: {slice_k} of K for {lanes} lanes of 16-byte vectors"
        return None

    def priority(
        self, config: KernelConfig, problem: Problem, caps: DeviceCaps
    ) -> tuple[float, ...]:
        """Rank survivors for the budget.

        GEMM tiles: (1) the DMA pipeline, which measured ahead of the
        register-staged one at every fp16/bf16 shape tried; (2) the time
        :func:`gemm_time_estimate` gives; (3) fewer split-K programs per
        tile; (4) more stages in flight; (5) waves: 8 for DMA tiles of at
        least 128x128, or 64x64 when split (two waves per SIMD hide LDS
        latency), else 4, and fewer for register-staged tiles (more registers
        each); (6) the taller of two
        transposed tiles; (7) least padding waste.
        GEMV strips: HBM-bound, so (1) one round of workgroups (a second
        round doubles some CUs' streams), (2) as many workgroups as that
        round allows, (3) strips of at least 512 bytes per row (narrower
        pieces share 128-byte lines between workgroups, whose CUs then fetch
        them twice), (4) eight waves (the most bytes in flight per CU), (5)
        fewer slices (a shorter cross-slice tail). Measured at 1x11008x4096
        bf16 (kernel-only): 172 workgroups of 512-byte strips stream at 97%
        of 256 workgroups' rate, while 256-byte and 128-byte strips and grids
        past one round are slower. GEMV candidates sort ahead of MFMA tiles
        for decode shapes.
        """
        dims = problem.dims_dict
        programs = self.num_programs(config, problem)
        if config.get("GEMV") and problem.layout == "bt":
            # gemv_dot measured best with whole 64-lane columns and no split
            # wherever that fills the CUs (1x11008x4096 bf16: 18.4 us against
            # 32 us for the strip kernel's tuned configuration).
            lanes = config.get("LANES_PER_ROW", GEMV_DEFAULT_LANES_PER_ROW)
            return (0, -min(programs, caps.cu_count), config["SPLIT_K"], -lanes,
                    abs(config["num_warps"] - 4))
        if config.get("GEMV"):
            lanes = config.get("LANES_PER_ROW", GEMV_DEFAULT_LANES_PER_ROW)
            return (
                0,
                programs > caps.cu_count,
                -min(programs, caps.cu_count),
                -min(lanes * VECTOR_BYTES, 512),
                abs(config["num_warps"] - 8),
                config["SPLIT_K"],
            )
        bm, bn = config["BLOCK_M"], config["BLOCK_N"]
        direct = config.get("DIRECT", 0)
        split = config.get("SPLIT_K", 1)
        estimate = gemm_time_estimate(config, problem, caps)
        padded = ceil_div(dims["M"], bm) * bm * ceil_div(dims["N"], bn) * bn
        waste = padded / (dims["M"] * dims["N"])
        if direct:
            wide = bm * bn >= 128 * 128 or (split > 1 and bm * bn >= 64 * 64)
            wave_rank = abs(config["num_warps"] - (8 if wide else 4))
        elif itemsize(problem.dtype) == 4 and bm * bn >= 256 * 128:
            # fp32 on the staged pipeline: a 256x128 tile measured 136 TFLOP/s
            # at 8 waves against 112 at 4 (4096^3); eight waves hide the
            # fp32 MFMAs' longer issue better than the registers they cost.
            wave_rank = abs(config["num_warps"] - 8)
        else:
            wave_rank = config["num_warps"]
        return (
            1,
            -direct,
            round(estimate * 1e6, 2),
            split,
            -config["num_stages"],
            wave_rank,
            bm < bn,
            waste,
        )


#: Reuse ``BM*BN/(BM+BN)`` of the 256x128 tile, the largest the DMA pipeline
#: instantiates; the GEMM estimate treats it as the full MFMA rate.
_FULL_RATE_REUSE = 256 * 128 / (256 + 128)
#: Start-up and wind-down of one program's K loop, in k-slices of work: what
#: makes splitting K into short ranges cost more than it saves.
_PIPELINE_FILL_SLICES = 3
#: MI355X rates the estimate is calibrated on (fp16, cache flushed): the
#: 256x128 DMA tile sustains about 1.0 PFLOP/s over 256 CUs; streaming
#: kernels reach about 5 TB/s of HBM; a program whose slices are latency-bound
#: (few rows) advances about one 64-wide k-slice per 0.35 us.
_CU_FLOPS = 1.0e15 / 256
_HBM_BYTES_PER_S = 5.0e12
_SLICE_LATENCY_S = 0.35e-6
#: Waves one CU holds (8 per SIMD), for co-resident workgroups.
_WAVES_PER_CU = 32


#: CUs per XCD on MI355X: the workgroups one XCD's L2 serves at a time.
_CUS_PER_XCD = 32


def gemm_group_m(block_m: int, block_n: int) -> int:
    """Band height (GROUP_M) that makes each XCD's concurrent tiles a near-square block.

    Workgroups are dispatched to the 8 XCDs round-robin and the kernels regroup
    them so that each XCD takes a contiguous run of tile indices; within a
    band of GROUP_M tile rows consecutive indices walk down the band. One
    XCD's 32 concurrent tiles then cover GROUP_M rows of A tiles and
    32/GROUP_M columns of B tiles, and its L2 fetches
    ``GROUP_M*BM + (32/GROUP_M)*BN`` rows of K per k-slice, least at
    ``GROUP_M = sqrt(32*BN/BM)`` (rounded to a power of two). Measured on
    MI355X: the 256x128 tile at 2048x4096x4096 runs in the same time at
    GROUP_M 2..16 and fetches 160 MiB from beyond L2 at GROUP_M=8 (each XCD
    reads all of A) but 128 MiB at 4; the fused 4096x11008x4096 launch fetches
    1004 MiB at 8 and 729 MiB at 4.
    """
    ideal = math.sqrt(_CUS_PER_XCD * block_n / block_m)
    return int(min(16, max(1, 2 ** math.floor(math.log2(ideal) + 0.5))))


def gemm_resident_workgroups(config: KernelConfig, caps: DeviceCaps, elem: int = 2) -> int:
    """Workgroups of one MFMA-tile config a CU holds at once (LDS and waves)."""
    bm, bn = config["BLOCK_M"], config["BLOCK_N"]
    stages = config.get("num_stages", 2)
    if config.get("DIRECT"):
        lds = gemm_direct_lds_bytes(bm, bn, stages)
    else:
        lds = gemm_lds_bytes(bm, bn, config["BLOCK_K"], stages, elem)
    return max(1, min(caps.lds_per_cu // max(lds, 1), _WAVES_PER_CU // config["num_warps"]))


def gemm_time_estimate(config: KernelConfig, problem: Problem, caps: DeviceCaps) -> float:
    """Seconds one MFMA-tile GEMM launch should take, from three bounds.

    * compute: each CU runs ``ceil(workgroups / CUs)`` tiles back to back,
      each ``BM*BN*64*2`` FLOP per k-slice (plus the pipeline's fill) at the
      rate its reuse ``BM*BN/(BM+BN)`` sustains, ``sqrt(reuse / reuse_256x128)``
      of the full rate; with several rounds of tiles only the last, partial
      round is split, so its programs are shorter;
    * memory: the operands once, C once, and with split-K every program's
      fp32 partial tile written and read back, at streaming HBM rate;
    * latency: few-row tiles wait on each k-slice's DMA; co-resident
      workgroups (as LDS and waves allow) wait together.

    Calibrated on MI355X measurements: over the 50 tuned fp16 shapes from
    M=16 to 4096 its first candidate measures 4% above the tuned winner on
    average (19% at worst); it ranks the one-pass
    256x128 tile first on large problems, a split last round at
    4096x11008x4096, and split 32x64..128x128 tiles at M=16..256.
    """
    dims = problem.dims_dict
    m, n, k = dims["M"], dims["N"], dims["K"]
    bm, bn, bk = config["BLOCK_M"], config["BLOCK_N"], config["BLOCK_K"]
    split = config.get("SPLIT_K", 1)
    elem = itemsize(problem.dtype)
    tiles = ceil_div(m, bm) * ceil_div(n, bn)
    resident = gemm_resident_workgroups(config, caps, elem)
    round_ = caps.cu_count * resident
    # With several rounds of tiles only the last, partial round is split.
    whole = tiles // round_ * round_ if split > 1 and tiles >= round_ else (0 if split > 1 else tiles)
    split_programs = (tiles - whole) * split
    all_slices = ceil_div(k, bk) + _PIPELINE_FILL_SLICES
    split_slices = ceil_div(ceil_div(k, bk), split) + _PIPELINE_FILL_SLICES
    reuse = min((bm * bn) / (bm + bn), _FULL_RATE_REUSE)
    rate = _CU_FLOPS * math.sqrt(reuse / _FULL_RATE_REUSE)
    tile_flops = bm * bn * bk * 2
    compute = (ceil_div(whole, caps.cu_count) * all_slices
               + ceil_div(split_programs, caps.cu_count) * split_slices) * tile_flops / rate
    moved = (m * k + k * n + m * n) * elem + 2 * split_programs * bm * bn * 4 * (split > 1)
    memory = moved / _HBM_BYTES_PER_S
    latency = (ceil_div(whole, round_) * all_slices
               + ceil_div(split_programs, round_) * split_slices) * _SLICE_LATENCY_S
    # A 4-norm rather than the plain maximum: the largest bound decides, and a
    # config with slack in the other two ranks ahead of one without.
    return (compute**4 + memory**4 + latency**4) ** 0.25


class MatmulSearchSpace(_GemmSpace):
    operation = "matmul"


class FusedLinearSearchSpace(_GemmSpace):
    operation = "fused_linear"


def gemm_instantiations(
    caps: DeviceCaps | None = None, *, direct: int = 0
) -> dict[int, list[tuple[int, ...]]]:
    """Tile configs the build compiles for one pipeline, keyed by element size.

    Every (BLOCK_M, BLOCK_N, BLOCK_K, num_warps, num_stages) point of the
    GEMM grid that passes the shape-independent rules.
    """
    from kernelforge.runtime.env import MI355X_CAPS

    caps = caps if caps is not None else MI355X_CAPS
    space = _GemmSpace
    out: dict[int, list[tuple[int, ...]]] = {}
    for elem in (2, 4):
        out[elem] = [
            (bm, bn, bk, w, s)
            for bm, bn, bk, w, s in product(
                space.BLOCK_M, space.BLOCK_N, space.BLOCK_K, space.NUM_WARPS, space.NUM_STAGES
            )
            if gemm_instantiation_reason(bm, bn, bk, w, s, elem, caps, direct=direct) is None
        ]
    return out


# ---------------------------------------------------------------------------
# Row kernels (softmax, rmsnorm): one pass, whole row in registers.
# ---------------------------------------------------------------------------


class _RowReductionSpace(SearchSpace):
    """Shared by softmax and rmsnorm.

    BLOCK_SIZE is fixed by the row width (the row must fit), which leaves the
    wave count and the rows per workgroup free (search.py:422-503).
    """

    NUM_WARPS = (1, 2, 4, 8, 16)
    ROWS_PER_PROGRAM = (1, 2, 4, 8)

    #: fp32 values a lane holds for its share of the row: at most 64 (with
    #: RMSNorm's gamma copy, 128 of a lane's registers).
    MIN_ELEMS_PER_LANE = 1
    MAX_ELEMS_PER_LANE = 64

    #: Widest single-pass row: 16384 fp32 values (64 KiB) per workgroup in
    #: registers. At 16 waves (1024 lanes, the workgroup limit) each lane may
    #: use 128 registers, which holds 16 values plus gamma and addresses; the
    #: kernels' launch bounds allow 16384/EPT lanes, so EPT=64 runs at <= 4
    #: waves with 512 registers per lane. The default configuration uses 16
    #: waves at this width. The value equals the reference's single-pass
    #: limit (search.py:441-459), re-derived from the gfx950 register file.
    MAX_WAVES = 16
    MAX_BLOCK_SIZE = 16384

    def grid(self, problem: Problem) -> Iterator[KernelConfig]:
        block = next_power_of_2(problem.dims_dict["cols"])
        for warps, rows in product(self.NUM_WARPS, self.ROWS_PER_PROGRAM):
            yield KernelConfig(
                self.operation, BLOCK_SIZE=block, ROWS_PER_PROGRAM=rows, num_warps=warps
            )

    def num_programs(self, config: KernelConfig, problem: Problem) -> int:
        return ceil_div(problem.dims_dict["rows"], config["ROWS_PER_PROGRAM"])

    def reject_reason(self, config: KernelConfig, problem: Problem, caps: DeviceCaps) -> str | None:
        block = config["BLOCK_SIZE"]
        if block > self.MAX_BLOCK_SIZE:
            return f"row of {problem.dims_dict['cols']} exceeds the single-pass limit"
        lanes = config["num_warps"] * caps.wave_size
        if lanes > caps.max_threads_per_workgroup:
            return f"workgroup size: {lanes} lanes exceeds {caps.max_threads_per_workgroup}"
        per_lane = block / lanes
        if per_lane < self.MIN_ELEMS_PER_LANE:
            return f"idle lanes: {lanes} lanes for BLOCK_SIZE={block}"
        if per_lane > self.MAX_ELEMS_PER_LANE:
            return f"register pressure: {per_lane:.0f} elements per lane"
        rows = problem.dims_dict["rows"]
        if config["ROWS_PER_PROGRAM"] > rows:
            return f"ROWS_PER_PROGRAM={config['ROWS_PER_PROGRAM']} exceeds {rows} rows"
        return None

    def priority(
        self, config: KernelConfig, problem: Problem, caps: DeviceCaps
    ) -> tuple[float, ...]:
        """Fill the CUs first, then 8-16 elements per lane (two 16-byte loads in
        flight per lane), then fewer rows per program."""
        programs = min(self.num_programs(config, problem), caps.cu_count)
        per_lane = config["BLOCK_SIZE"] / (config["num_warps"] * caps.wave_size)
        return (-programs, abs(per_lane - 12), config["ROWS_PER_PROGRAM"])


class SoftmaxSearchSpace(_RowReductionSpace):
    operation = "softmax"


#: Bytes of a row the two-pass RMSNorm may keep in LDS between its passes:
#: 160 KiB per workgroup on gfx950 less room for the reduction buffer
#: (csrc/wide_rows.hip, kMaxStagedBytes).
TWO_PASS_MAX_STAGED_BYTES = 159 * 1024


def two_pass_block(warps: int, unroll: int, elem: int) -> int:
    """Columns one trip of the two-pass RMSNorm covers: a 16-byte vector per
    lane, ``unroll`` times."""
    return warps * 64 * (VECTOR_BYTES // elem) * unroll


class RMSNormSearchSpace(_RowReductionSpace):
    """The single-pass grid plus the two-pass kernel as an algorithmic axis.

    The reference lists the two-pass variant as its first future improvement
    (README.md:656-660): it lifts the 16384-column cap and gives the space a
    choice of algorithm, not only of tuning. A two-pass point is
    ``TWO_PASS=1`` with BLOCK_SIZE = columns per trip (``TWO_PASS_UNROLL``
    16-byte vectors per lane), and ``STAGE_ROW`` = 1 to keep the row in LDS
    between the passes so HBM sees it once.
    """

    operation = "rmsnorm"
    TWO_PASS_WARPS = (4, 8, 16)
    TWO_PASS_UNROLL = (1, 2, 4, 8)
    TWO_PASS_ROWS_PER_PROGRAM = (1, 2, 4)
    STAGE_ROW = (1, 0)

    def grid(self, problem: Problem) -> Iterator[KernelConfig]:
        yield from super().grid(problem)
        elem = itemsize(problem.dtype)
        for warps, unroll, rows, stage in product(
            self.TWO_PASS_WARPS, self.TWO_PASS_UNROLL, self.TWO_PASS_ROWS_PER_PROGRAM,
            self.STAGE_ROW,
        ):
            yield KernelConfig(
                self.operation,
                TWO_PASS=1,
                BLOCK_SIZE=two_pass_block(warps, unroll, elem),
                ROWS_PER_PROGRAM=rows,
                STAGE_ROW=stage,
                num_warps=warps,
            )

    def reject_reason(self, config: KernelConfig, problem: Problem, caps: DeviceCaps) -> str | None:
        if not config.get("TWO_PASS"):
            return super().reject_reason(config, problem, caps)
        d = problem.dims_dict
        elem = itemsize(problem.dtype)
        warps = config["num_warps"]
        lanes = warps * caps.wave_size
        if lanes > caps.max_threads_per_workgroup:
            return f"workgroup size: {lanes} lanes exceeds {caps.max_threads_per_workgroup}"
        unroll = config["BLOCK_SIZE"] // two_pass_block(warps, 1, elem)
        # x and gamma for `unroll` vectors per lane: 8 of each need more than
        # the 128 registers a lane has at 16 waves.
        if unroll >= 8 and warps > 8:
            return f"register pressure: {unroll} vectors per lane allow at most 8 waves, got {warps}"
        row_bytes = d["cols"] * elem
        if config.get("STAGE_ROW") and row_bytes > TWO_PASS_MAX_STAGED_BYTES:
            return (
                f"LDS: a staged row of {row_bytes // 1024} KiB exceeds "
                f"{TWO_PASS_MAX_STAGED_BYTES // 1024} KiB"
            )
        smallest = two_pass_block(min(self.TWO_PASS_WARPS), 1, elem)
        if config["BLOCK_SIZE"] > max(next_power_of_2(d["cols"]), smallest):
            return f"idle lanes: a trip of {config['BLOCK_SIZE']} columns for a row of {d['cols']}"
        if config["ROWS_PER_PROGRAM"] > d["rows"]:
            return f"ROWS_PER_PROGRAM={config['ROWS_PER_PROGRAM']} exceeds {d['rows']} rows"
        return None

    def priority(
        self, config: KernelConfig, problem: Problem, caps: DeviceCaps
    ) -> tuple[float, ...]:
        """Single-pass first where it fits (it reads the row once, from
        registers); two-pass after it, staged rows first, then 2-4 vectors in
        flight per lane."""
        if not config.get("TWO_PASS"):
            return (0, *super().priority(config, problem, caps))
        programs = min(self.num_programs(config, problem), caps.cu_count)
        unroll = config["BLOCK_SIZE"] // two_pass_block(config["num_warps"], 1, itemsize(problem.dtype))
        return (
            1, -programs, -config.get("STAGE_ROW", 0), abs(unroll - 3), -config["num_warps"],
            config["ROWS_PER_PROGRAM"],
        )


def default_row_config(operation: str, n_cols: int, dtype=None) -> KernelConfig:
    """One wave per 512 columns, up to 16 waves; one row per workgroup.

    For RMSNorm rows beyond the single-pass limit: the two-pass kernel at 8
    waves and 8192 columns per trip (valid for every dtype: four fp32 or two
    16-bit vectors per lane), with the row staged in LDS when it fits there
    at ``dtype``'s width (fp32 when no dtype is given).
    """
    block = next_power_of_2(n_cols)
    if operation == "rmsnorm" and block > _RowReductionSpace.MAX_BLOCK_SIZE:
        elem = itemsize(dtype) if dtype is not None else 4
        return KernelConfig(
            operation,
            TWO_PASS=1,
            BLOCK_SIZE=8192,
            ROWS_PER_PROGRAM=1,
            STAGE_ROW=int(n_cols * elem <= TWO_PASS_MAX_STAGED_BYTES),
            num_warps=8,
        )
    warps = max(1, min(_RowReductionSpace.MAX_WAVES, block // 512))
    return KernelConfig(operation, BLOCK_SIZE=block, ROWS_PER_PROGRAM=1, num_warps=warps)


class VectorAddSearchSpace(SearchSpace):
    """Elementwise: nothing to tile or reuse (search.py:514-539 in the reference).

    BLOCK_SIZE elements per workgroup of ``num_warps`` waves; a lane holds
    BLOCK_SIZE / lanes of them, a power of two from 1 to 64 (the compiled
    set), loaded 16 bytes at a time where that many fit.
    """

    operation = "vector_add"
    BLOCK_SIZE = (256, 512, 1024, 2048, 4096, 8192, 16384)
    NUM_WARPS = (1, 2, 4, 8, 16)
    MAX_ELEMS_PER_LANE = 64

    def grid(self, problem: Problem) -> Iterator[KernelConfig]:
        for block, warps in product(self.BLOCK_SIZE, self.NUM_WARPS):
            yield KernelConfig(self.operation, BLOCK_SIZE=block, num_warps=warps)

    def num_programs(self, config: KernelConfig, problem: Problem) -> int:
        return ceil_div(problem.dims_dict["n"], config["BLOCK_SIZE"])

    def reject_reason(self, config: KernelConfig, problem: Problem, caps: DeviceCaps) -> str | None:
        lanes = config["num_warps"] * caps.wave_size
        if lanes > caps.max_threads_per_workgroup:
            return f"workgroup size: {lanes} lanes exceeds {caps.max_threads_per_workgroup}"
        per_lane = config["BLOCK_SIZE"] / lanes
        if per_lane < 1:
            return f"idle lanes: {lanes} lanes for BLOCK_SIZE={config['BLOCK_SIZE']}"
        if per_lane > self.MAX_ELEMS_PER_LANE:
            return f"register pressure: {per_lane:.0f} elements per lane"
        return None

    def priority(
        self, config: KernelConfig, problem: Problem, caps: DeviceCaps
    ) -> tuple[float, ...]:
        """Fill the CUs, then whole 16-byte loads, then 64 bytes per lane and
        operand (four loads of each input in flight), then larger workgroups."""
        programs = min(self.num_programs(config, problem), caps.cu_count)
        lane_bytes = config["BLOCK_SIZE"] // (config["num_warps"] * caps.wave_size) * itemsize(
            problem.dtype
        )
        partial = 1 if lane_bytes < VECTOR_BYTES else 0
        return (-programs, partial, abs(lane_bytes.bit_length() - 7), -config["num_warps"])


SEARCH_SPACES: dict[str, type[SearchSpace]] = {
    "vector_add": VectorAddSearchSpace,
    "softmax": SoftmaxSearchSpace,
    "matmul": MatmulSearchSpace,
    "rmsnorm": RMSNormSearchSpace,
    "fused_linear": FusedLinearSearchSpace,
}


def search_space(operation: str, **kwargs) -> SearchSpace:
    try:
        return SEARCH_SPACES[operation](**kwargs)
    except KeyError:
        raise ValueError(
            f"no search space for {operation!r}; known: {sorted(SEARCH_SPACES)}"
        ) from None
