"""The command line, in process (kernelforge/tests/test_cli.py).

Parsing, shape resolution and the commands that need no GPU run everywhere;
the commands that launch kernels are marked ``gpu`` (the benchmark/report
pipeline is exercised end to end in test_gpu_widening.py).
"""

from __future__ import annotations

import pytest
import torch

from kernelforge.cli.main import OPERATIONS, build_parser, build_problem, main


def parse(argv: list[str]):
    return build_parser().parse_args(argv)


def test_every_operation_is_offered_by_the_cli():
    from kernelforge.kernels import operator_names

    assert set(OPERATIONS) == set(operator_names())


def test_version_flag_exits_cleanly(capsys):
    with pytest.raises(SystemExit) as exit_info:
        main(["--version"])
    assert exit_info.value.code == 0
    assert "kernelforge" in capsys.readouterr().out


def test_missing_subcommand_and_unknown_operation_are_parser_errors():
    with pytest.raises(SystemExit):
        parse([])
    with pytest.raises(SystemExit):
        parse(["tune", "flash_attention"])
    with pytest.raises(SystemExit):
        parse(["tune", "matmul", "--dtype", "fp8"])
    with pytest.raises(SystemExit):
        parse(["benchmark", "matmul", "--suite", "correctness"])  # a test-only suite


def test_shape_flags_map_to_named_dimensions():
    p = build_problem("matmul", parse(["tune", "matmul", "-m", "512", "-n", "1024", "-k", "256"]))
    assert p.dims_dict == {"M": 512, "N": 1024, "K": 256} and p.dtype is torch.float16
    p = build_problem("rmsnorm", parse(["tune", "rmsnorm", "--rows", "128", "--cols", "768",
                                         "--dtype", "bf16"]))
    assert p.dims_dict == {"rows": 128, "cols": 768} and p.dtype is torch.bfloat16
    # --n means N for a GEMM, so the element count has its own flag.
    p = build_problem("vector_add", parse(["tune", "vector_add", "--elements", "1000003"]))
    assert p.dims_dict == {"n": 1000003}


@pytest.mark.parametrize("operation", OPERATIONS)
def test_defaults_produce_a_valid_problem(operation):
    problem = build_problem(operation, parse(["tune", operation]))
    assert problem.operation == operation
    assert all(value > 0 for value in problem.dims_dict.values())


def test_env_runs_without_a_gpu(capsys):
    assert main(["env"]) == 0
    out = capsys.readouterr().out
    assert "PyTorch" in out and "Device limits" in out
    if not torch.cuda.is_available():
        assert "No ROCm device" in out


def test_explain_reports_the_search_space_without_a_gpu(capsys):
    assert main(["tune", "matmul", "-m", "2048", "-n", "4096", "-k", "4096", "--explain"]) == 0
    out = capsys.readouterr().out
    assert "grid points" in out and "selected (budget)" in out
    assert main(["tune", "vector_add", "--elements", "67108864", "--explain"]) == 0
    assert "grid points      : 35" in capsys.readouterr().out


def test_kernel_commands_fail_clearly_without_a_gpu(capsys):
    if torch.cuda.is_available():
        pytest.skip("this is the no-GPU error path")
    for argv in (["tune", "matmul", "--no-db", "--no-cache"],
                 ["benchmark", "softmax", "--suite", "smoke", "--no-db", "--no-cache"],
                 ["compare", "transformer", "--seq", "1", "--no-cache"],
                 ["profile", "rmsnorm", "--no-cache"]):
        assert main(argv) == 1, argv
        assert "ROCm GPU" in capsys.readouterr().err


def test_report_without_a_database_is_an_error(capsys, tmp_path):
    assert main(["report", "--db", str(tmp_path / "missing.db")]) == 2
    assert "no results database" in capsys.readouterr().err


def test_cache_list_and_clear(capsys, tmp_path):
    from kernelforge.tuning.cache import ConfigCache
    from kernelforge.tuning.config import KernelConfig, Problem

    path = tmp_path / "configs.json"
    assert main(["cache", "list", "--cache", str(path)]) == 0
    assert "0 entry(ies)" in capsys.readouterr().out
    ConfigCache(path).put(Problem.create("vector_add", "fp32", n=64), "dev",
                          KernelConfig("vector_add", BLOCK_SIZE=256, num_warps=1))
    assert main(["cache", "clear", "--cache", str(path)]) == 0
    assert "removed 1" in capsys.readouterr().out


@pytest.mark.gpu
def test_tune_runs_end_to_end_and_writes_both_stores(capsys, tmp_path):
    db_path, cache_path = tmp_path / "results.db", tmp_path / "configs.json"
    code = main(["tune", "rmsnorm", "--rows", "512", "--cols", "1024", "--iterations", "20",
                 "--warmup", "5", "--db", str(db_path), "--cache", str(cache_path)])
    assert code == 0
    out = capsys.readouterr().out
    assert "passed correctness" in out and "Best configuration" in out
    assert db_path.exists() and cache_path.exists()


@pytest.mark.gpu
def test_compare_runs_end_to_end(capsys):
    code = main(["compare", "vector_add", "--elements", "1000003", "--iterations", "20",
                 "--warmup", "5", "--no-db", "--no-cache"])
    assert code == 0
    out = capsys.readouterr().out
    assert "kernelforge" in out and "torch_eager" in out and "GB/s" in out


def test_b_layout_flag_names_the_k_contiguous_problem():
    """``--b-layout nk`` tunes the nn.Linear-weight layout, keyed ``+bt``."""
    import argparse

    from kernelforge.cli.main import build_problem

    args = argparse.Namespace(dtype="bf16", m=1, n=11008, k=4096, b_layout="nk")
    assert build_problem("matmul", args).cache_key == "matmul/bf16/1x11008x4096+bt"
    args.b_layout = "kn"
    assert build_problem("matmul", args).cache_key == "matmul/bf16/1x11008x4096"
    with pytest.raises(ValueError, match="b-layout"):
        build_problem("rmsnorm", argparse.Namespace(dtype="fp32", rows=4, cols=8, b_layout="nk"))
