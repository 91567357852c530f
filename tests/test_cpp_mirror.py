"""The C++ mirror of the reference's Tensor-level interface
(candle-3d_amd/host/lux3d_candle.hpp) and the reference's own known-answer
tests restated against it (tests/cpp/test_reference_kats.cpp, built by
__graft_entry__.build() / `make -C tests/cpp`).

On the CPU only the host-side argument checks run (`--cpu`); the GPU test
runs every case through liblux3d_fused on the device.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_reference_kats")


def _run(args, timeout):
    assert os.path.exists(BIN), f"{BIN} is not built (run __graft_entry__.build() or make -C tests/cpp)"
    p = subprocess.run([BIN] + args, capture_output=True, text=True, timeout=timeout)
    print(p.stdout, p.stderr, flush=True)
    return p


def test_cpp_mirror_host_checks():
    p = _run(["--cpu"], 60)
    assert p.returncode == 0
    assert "PASS errors_on_host" in p.stdout


@pytest.mark.gpu
def test_cpp_mirror_reference_kats_on_gpu():
    p = _run([], 120)
    assert p.returncode == 0, p.stdout
    assert "0 failures" in p.stdout
    for case in ("rope_tables_match_reference_formula", "qk_rms_norm_matches_reference",
                 "timestep_embedding_matches_reference", "dinov3_rope_applies_to_patches_only"):
        assert f"PASS {case}" in p.stdout
