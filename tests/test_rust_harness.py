"""The Rust harness files, checked without a Rust toolchain: the parity/bench
script's command lines (a stand-in `cargo` on PATH echoes its arguments), the
example's options against the script's, and the parity test names the script
runs against those the test file defines."""

import os
import re
import stat
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUST = os.path.join(REPO, "candelora-metal-kernels_amd", "rust")
SCRIPT = os.path.join(RUST, "run_iq_parity_bench.sh")


@pytest.fixture()
def fake_cargo(tmp_path):
    cargo = tmp_path / "cargo"
    cargo.write_text('#!/bin/sh\necho "cargo $*"\n')
    cargo.chmod(cargo.stat().st_mode | stat.S_IEXEC)
    env = dict(os.environ)
    env["PATH"] = f"{tmp_path}{os.pathsep}{env.get('PATH', '')}"
    return env


def _run(env, *args):
    return subprocess.run(["bash", SCRIPT, *args], env=env, capture_output=True, text=True)


def _cargo_lines(out):
    return [l for l in out.splitlines() if l.startswith("cargo ")]


def test_hip_backend_runs_hip_tests_and_rocm_bench(fake_cargo):
    r = _run(fake_cargo, "--backend", "hip", "--variants", "iq2-xxs, IQ3-S", "--m", "4")
    assert r.returncode == 0, r.stderr
    lines = _cargo_lines(r.stdout)
    assert lines[:2] == ["cargo test -q --features rocm cpu_vs_hip_parity_iq2_xxs",
                         "cargo test -q --features rocm cpu_vs_hip_parity_iq3_s"]
    assert lines[2] == ("cargo run --release --features rocm --example iq2_matmul_bench -- "
                        "--backend hip --variants iq2-xxs,iq3-s --m 4 --out-dim 4096 "
                        "--in-dim 4096 --warmup-runs 5 --runs 20 --dtype f16 "
                        "--activation-quant-mode off")


def test_metal_backend_is_the_default_and_w8a8_names(fake_cargo):
    r = _run(fake_cargo, "--activation-quant-mode", "W8A8", "--skip-bench")
    assert r.returncode == 0, r.stderr
    assert _cargo_lines(r.stdout) == [
        f"cargo test -q --features metal cpu_vs_metal_parity_w8a8_{v}"
        for v in ("iq2_xxs", "iq2_xs", "iq2_s", "iq3_s")]


@pytest.mark.parametrize("args", [["--backend", "cuda"], ["--variants", "iq4-nl"],
                                  ["--activation-quant-mode", "w4a8"], ["--bogus"], ["--m"]])
def test_bad_arguments_fail(fake_cargo, args):
    r = _run(fake_cargo, *args)
    assert r.returncode != 0
    assert not _cargo_lines(r.stdout)


def test_example_accepts_every_option_the_script_passes():
    src = open(os.path.join(RUST, "examples", "iq2_matmul_bench.rs")).read()
    script = open(SCRIPT).read()
    example_args = script.split("--example iq2_matmul_bench --", 1)[1]
    passed = set(re.findall(r"(--[a-z-]+) \"\$\{", example_args))
    handled = set(re.findall(r'"(--[a-z-]+)" =>', src))
    assert passed and passed <= handled, passed - handled
    assert '#[path = "support/backend.rs"]' in src
    assert os.path.exists(os.path.join(RUST, "examples", "support", "backend.rs"))


def test_hip_parity_test_names_exist():
    tests = open(os.path.join(RUST, "src", "hip", "parity_tests.rs")).read()
    defined = set(re.findall(r"fn (cpu_vs_hip_parity_\w+)\(", tests))
    for mode in ("", "w8a8_"):
        for v in ("iq2_xxs", "iq2_xs", "iq2_s", "iq3_s"):
            assert f"cpu_vs_hip_parity_{mode}{v}" in defined
