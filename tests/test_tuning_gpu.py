"""Measured tuner on the GPU (tests/correctness/tuning.rs:10-41 plus the
persistent store, src/pipeline/tuning.rs:98-199)."""

import os

import numpy as np
import pytest

from test_gemm_gpu import check_f32

pytestmark = pytest.mark.gpu


@pytest.fixture
def cache_dir(tmp_path, monkeypatch):
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path))
    return tmp_path


def store_lines(cache_dir):
    files = list((cache_dir / "tensor-ash").glob("tuned_kernels_*.txt"))
    assert len(files) == 1, files
    lines = files[0].read_text().splitlines()
    assert lines[0].startswith("tensor-ash-tune-v3 hip=") and "arch=gfx950" in lines[0]
    return lines[1:]


def test_tune_shape_then_compute_is_correct(ta, ctx, oracle, cache_dir):
    ex = ta.Executor(ctx, tune=False)
    m, n, k = 320, 192, 448
    ex.tune_shape(1, m, n, k)
    lines = store_lines(cache_dir)
    assert len(lines) == 1 and lines[0].startswith(f"1 {m} {n} {k} ")
    winner = lines[0].split()[4]
    assert winner in ta.kernel_names()
    assert ex.dispatch_info_for(1, m, n, k)["kernel"] == winner
    ha, hb = oracle.fill_det(m * k, 91), oracle.fill_det(k * n, 92)
    a, b, c = ex.tensor_from(ha, shape=[m, k]), ex.tensor_from(hb, shape=[k, n]), ex.tensor([m, n])
    ex.matmul(a, b, c)
    check_f32(ex.download(c), oracle.cpu_bmm(ha, hb, None, 1, m, n, k), k, oracle, epi=False)
    ex.tune_shape(1, m, n, k)  # already recorded: no-op
    assert store_lines(cache_dir) == lines
    # a fresh executor picks the persisted winner up
    ex2 = ta.Executor(ctx, tune=False)
    assert ex2.dispatch_info_for(1, m, n, k)["kernel"] == winner


def test_online_tuning_on_first_plain_op(ta, ctx, oracle, cache_dir):
    """ML_TUNE semantics (dispatch.rs:114-149): the first plain op of a new
    shape is measured (including the split-K probe on deep-K, few-tile
    shapes) and the result stays correct."""
    ex = ta.Executor(ctx, tune=True)
    m, n, k = 64, 128, 8192
    ha, hb = oracle.fill_det(m * k, 5), oracle.fill_det(k * n, 6)
    a, b, c = ex.tensor_from(ha, shape=[m, k]), ex.tensor_from(hb, shape=[k, n]), ex.tensor([m, n])
    ex.matmul(a, b, c)
    check_f32(ex.download(c), oracle.cpu_bmm(ha, hb, None, 1, m, n, k), k, oracle, epi=False)
    lines = store_lines(cache_dir)
    assert any(l.startswith(f"1 {m} {n} {k} ") for l in lines)
    # the tuned route (DP kernel or split-K) still matches the oracle
    ex.matmul(a, b, c)
    check_f32(ex.download(c), oracle.cpu_bmm(ha, hb, None, 1, m, n, k), k, oracle, epi=False)


def test_explicit_selection_skips_tuning(ta, ctx, cache_dir):
    ex = ta.Executor(ctx, kernel_selection="f32_m64n64", tune=True)
    ex.tune_shape(1, 128, 128, 128)
    assert not (cache_dir / "tensor-ash").exists()
    assert ex.dispatch_info_for(1, 128, 128, 128)["kernel"] == "f32_m64n64"


def test_stale_store_is_ignored(ta, ctx, cache_dir):
    d = cache_dir / "tensor-ash"
    d.mkdir()
    (d / "tuned_kernels_gfx950.txt").write_text("tensor-ash-tune-v3 hip=0 arch=gfx950 kernels=0\n"
                                                "1 4096 4096 4096 f32_m64n64\n")
    for name in os.listdir(d):
        (d / name).write_text("tensor-ash-tune-v3 stale header\n1 4096 4096 4096 f32_m64n64\n")
    ex = ta.Executor(ctx, tune=False)
    assert ex.dispatch_info_for(1, 4096, 4096, 4096)["kernel"] == "f32_m256n256"
