"""Index arithmetic of the prefill kernels, checked on the CPU with the
kernels' own code.

`prefill_fa_kernel<..., PAGED = true>` (tinyvllm_amd/csrc/flash_prefill.hip)
stages the block ids of a work-group's key range in LDS and maps every key a
K/V load touches -- padded rows of a partial tile and the re-requests of the
last tile included -- to a staged slot, through the `__host__ __device__`
functions of tinyvllm_amd/csrc/tv_paged_keys.h.  `paged_index_check.cpp`
compiles those functions for the host (hipcc, no GPU code) and checks every
slot for the shapes the GPU tests and the bench launch, for every kernel shape
(1 / 2 / 4 key groups, 32- / 64-key tiles).  A former clamp (to the last key of
the sequence instead of the last staged key) is planted through the driver and
must be caught.  The same driver checks the 128-row kernel's split causal
grids: units -> (query tile, key half) and the halves' key ranges.
"""

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
CSRC = HERE.parent / "tinyvllm_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

CASES = [
    # (q_len, start_pos, block_size, causal): the GPU tests' shapes and the bench's
    (100, 0, 16, True), (77, 300, 16, True), (256, 1000, 16, True), (64, 64, 4, True),
    (50, 200, 32, False), (512, 3584, 16, True), (16, 64, 16, True),
    (37, 0, 16, True), (50, 37, 16, True), (5, 87, 16, True), (33, 31, 128, True), (1, 4095, 1, True),
]


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    exe = tmp_path_factory.mktemp("paged_index") / "paged_index_check"
    res = subprocess.run([HIPCC, "-O1", "-std=c++17", f"-I{CSRC}", str(HERE / "paged_index_check.cpp"), "-o", str(exe)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    return exe


def run(exe, q_len, start, bs, causal, planted=False):
    args = [str(exe), str(q_len), str(start), str(bs), "1" if causal else "0"] + (["planted"] if planted else [])
    return subprocess.run(args, capture_output=True, text=True)


@pytest.mark.parametrize("q_len,start,bs,causal", CASES)
def test_every_touched_key_maps_to_a_staged_slot(checker, q_len, start, bs, causal):
    res = run(checker, q_len, start, bs, causal)
    assert res.returncode == 0 and res.stdout.startswith("ok "), res.stdout + res.stderr
    assert int(res.stdout.split()[1]) > 0


def test_the_old_clamp_reads_past_the_staged_table(checker):
    res = run(checker, 77, 300, 16, True, planted=True)
    assert res.returncode == 1 and "slot" in res.stdout, res.stdout + res.stderr


def test_split_units_cover_every_query_tile_once(checker):
    """The 128-row kernel's split grids (tinyvllm_amd/csrc/flash_prefill_rows.hip):
    every tile count up to 64 (L 8192) and every first split tile."""
    res = subprocess.run([str(checker), "split", "64"], capture_output=True, text=True)
    assert res.returncode == 0 and res.stdout.startswith("ok "), res.stdout + res.stderr


def test_overlapping_key_halves_are_caught(checker):
    res = subprocess.run([str(checker), "split", "8", "planted"], capture_output=True, text=True)
    assert res.returncode == 1 and "halves" in res.stdout, res.stdout + res.stderr
