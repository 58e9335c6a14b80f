"""The ggml backend add-on through its exported entry points, as llama.cpp
loads it (GGML_BACKEND_PATH -> ggml_backend_init): the C++ programs under
tests/cpp, one per reference test (tests/test-dispatch-gate.cpp,
test-memory-budget.cpp, test-mul-mat.cpp, test-host-ops.cpp,
test-safe-start.cpp, and the mul-mat-npu-nan/-fail ctest cases), and a seeded
sweep of random pieces (test_pieces_random).

Without a GPU the gate and the budget run under GGML_XDNA_PLAN_ONLY=1
(planning only); on the GPU they run for real, with the matmul, host-op and
failure programs. Each program prints PASS/FAIL lines and ALL PASS.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BIN = ROOT / "tests" / "cpp" / "_bin"
LIB = ROOT / "ggml-xdna_amd" / "libggml-zest.so"

SETTINGS = ("GGML_XDNA_PLAN_ONLY", "GGML_XDNA_HOST_ONLY", "GGML_XDNA_DEVICE", "GGML_XDNA_MAX_COPY_GB",
            "GGML_XDNA_FAIL_AFTER", "GGML_XDNA_NAN_AFTER", "GGML_XDNA_MIN_BATCH", "GGML_XDNA_MIN_MFLOP",
            "GGML_XDNA_BLOCKS", "GGML_XDNA_BLOCK_OPS", "GGML_XDNA_COPY_AT_LOAD", "GGML_XDNA_WRITE_ALL")


def run(prog: str, *args: str, timeout: int = 300, **env: str) -> str:
    exe = BIN / prog
    if not exe.exists():
        pytest.fail(f"{exe} is not built (run __graft_entry__.build())")
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    e = {k: v for k, v in os.environ.items() if k not in SETTINGS}
    e["GGML_BACKEND_PATH"] = str(LIB)
    e.update(env)
    print(f"[backend] {prog} {' '.join(args)} {env}", flush=True)
    r = subprocess.run([str(exe), *args], env=e, capture_output=True, text=True, timeout=timeout)
    out = r.stdout + r.stderr
    print(out, flush=True)
    assert r.returncode == 0 and "ALL PASS" in r.stdout, f"{prog} failed (exit {r.returncode}):\n{out}"
    return out


# ---- planning only: no GPU needed --------------------------------------------------

def test_dispatch_gate_planning():
    run("test_dispatch_gate", GGML_XDNA_PLAN_ONLY="1")


def test_memory_budget_planning():
    run("test_memory_budget", GGML_XDNA_PLAN_ONLY="1", GGML_XDNA_MAX_COPY_GB="0.05")


def test_safe_start_host_only():
    run("test_safe_start", "--host-only")


def test_two_contexts_on_threads_planning():
    run("test_contexts", GGML_XDNA_PLAN_ONLY="1", GGML_XDNA_MAX_COPY_GB="0.05")


def test_random_pieces_checker_self_check():
    # the random-piece test's CPU chain on sampled token rows (how it checks
    # its model-sized cases) equals the full chain on those rows; no GPU
    out = run("test_pieces_random", "--self-check", GGML_XDNA_PLAN_ONLY="1")
    assert "sampled rows equal" in out


def test_host_code_under_sanitizers():
    # the host side rebuilt with ThreadSanitizer and with AddressSanitizer +
    # UBSan (tests/cpp/Makefile, `sanitize`), the gate, budget, safe-start and
    # two-context programs run under each; any report or failure fails
    if not list((ROOT / "ggml-xdna_amd" / "_build").glob("*.hip.o")):
        pytest.fail("the kernel objects are not built (run __graft_entry__.build())")
    env = {k: v for k, v in os.environ.items() if k not in SETTINGS}
    r = subprocess.run(["make", "-s", "-C", str(ROOT / "tests" / "cpp"), "-j8", "sanitize-run"], env=env,
                       capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    print(out)
    assert r.returncode == 0, out
    assert out.count("ALL PASS") == 8, out


# ---- on the GPU ---------------------------------------------------------------------------

@pytest.mark.gpu
def test_dispatch_gate_gpu():
    out = run("test_dispatch_gate")
    assert "registration test multiply right" in out


@pytest.mark.gpu
def test_memory_budget_gpu():
    run("test_memory_budget", GGML_XDNA_MAX_COPY_GB="0.05")


@pytest.mark.gpu
def test_safe_start_no_such_gpu():
    run("test_safe_start")


@pytest.mark.gpu
def test_mul_mat_gpu():
    run("test_mul_mat")


@pytest.mark.gpu
def test_mul_mat_gpu_conversion_in_graph():
    # weight-cache entries built by the first graph instead of at load
    run("test_mul_mat", GGML_XDNA_COPY_AT_LOAD="0")


@pytest.mark.gpu
def test_host_ops_gpu():
    out = run("test_host_ops", GGML_XDNA_TRACE="2")
    # the FFN block's gate and up ran as one fused launch with the SwiGLU,
    # q, k and v as one grouped launch, and the down projection with the
    # residual ADD in its store
    assert "1 fused gate/up, 1 grouped, 1 with a residual add" in out


@pytest.mark.gpu
def test_random_pieces_gpu():
    # seeded random chains of norms, matmul groups, fused gate/up, residual
    # adds and in-place ops, every output against the same chain on the CPU;
    # the batch floor lowered so that ragged token counts down to 1 are taken
    run("test_pieces_random", "24", "1000", GGML_XDNA_MIN_BATCH="1")


@pytest.mark.gpu
def test_random_pieces_on_threads_gpu():
    # four backends computing on four threads at once, sharing the library,
    # the gate's reader log and the budget; each thread's tensor writes look
    # through every context's weight cache
    run("test_pieces_random", "6", "5000", "4", GGML_XDNA_MIN_BATCH="1")


@pytest.mark.gpu
def test_injected_failure_gpu():
    run("test_failure", GGML_XDNA_FAIL_AFTER="0")


@pytest.mark.gpu
def test_injected_nan_gpu():
    run("test_failure", GGML_XDNA_NAN_AFTER="0")
