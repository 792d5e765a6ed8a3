"""bench.py on the CPU: the one-GPU contract, the figures it reads from the
committed rocprofv3 summaries, and its useful-work count."""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402  (imports no GPU code at module level)


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}),
                                      ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused_with_a_message(argv, env):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + argv,
                       env={**os.environ, **env}, capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_profile_figures_parse():
    clock = bench.read_profile_value("bsattn_fwd_cfg3_clock.txt", "effective_clock_ghz")
    assert clock is not None and 1.0 < clock <= 2.4
    traffic = bench.read_traffic("bsattn_fwd_cfg3_traffic.txt")
    # At least the algorithmic bytes of a cfg3 launch (Q, K, V read once, the
    # output written once: 1.311e9), and no more than a few times that.
    assert traffic is not None and 1.311e9 <= traffic <= 4e9
    assert bench.read_profile_value("bsattn_fwd_cfg3_clock.txt", "no_such_key") is None
    assert bench.read_traffic("no_such_profile.txt") is None


def test_useful_flops_dense_closed_form():
    # Dense 3-tile plan at S = 300 (tiles of 128, 128, 44 rows): every query
    # against every key, 4 * d FLOP per pair.
    n = 3
    row_ptr = np.arange(0, n * n + 1, n)
    col_idx = np.tile(np.arange(n), n)
    assert bench.useful_tile_flops((row_ptr, col_idx), 300, heads=2) == 4 * 128 * 300 * 300 * 2


def test_useful_flops_sparse_against_token_count():
    rng = np.random.default_rng(7)
    S, n = 700, 6                        # last tile 60 rows
    bm = rng.random((n, n)) < 0.4
    bm[np.arange(n), np.arange(n)] = True
    row_ptr = np.concatenate([[0], np.cumsum(bm.sum(1))])
    col_idx = np.concatenate([np.flatnonzero(r) for r in bm])
    tok = np.minimum(128, S - 128 * np.arange(n))           # valid rows per tile
    pairs = sum(int(tok[q]) * int(tok[k]) for q in range(n) for k in range(n) if bm[q, k])
    assert bench.useful_tile_flops((row_ptr, col_idx), S, heads=3) == 4 * 128 * pairs * 3


def test_probe_library_loads_and_counts():
    """libch3probe.so (bench.py's same-run ceilings) loads on the host and its
    host-side bookkeeping matches the probe's loop: 8 waves x 4 chains x 4
    operand sets x 32,768 FLOP per 32x32x16 MFMA per iteration."""
    P = bench.probe_lib()
    assert P.h3probe_mfma_operand_bytes(256) == 256 * 512 * 8 * 16
    assert P.h3probe_mfma_flops(256, 2000) == 256 * 8 * 2000 * 4 * 4 * 32768.0
    # Argument checks refuse before touching the GPU.
    assert P.h3probe_mfma(2, None, 1, 1, None, None) == -1
    assert P.h3probe_stream(0, None, None, 17, 1, 4, None, None) == -1
    assert P.h3probe_stream(1, None, None, 16, 1, 3, None, None) == -1
