"""bench.py's host-side arithmetic, on the CPU: the algorithmic bytes per token of each KV
format, HBM bytes from the TCC request counters, the buffer-set count that keeps a kernel's
inputs out of the Infinity Cache, the copy-ceiling dispatch filter of the profile summary,
and the one-GPU guard."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_chain_bytes_per_token():
    # norm 4 x 2H; q, k read and written, v read, one table row; the cache rows
    norm = 4 * 2 * 2048
    qk = 2 * (2 * 16 * 128) + 2 * (2 * 4 * 128) + 2 * 4 * 128 + 2 * 128
    assert norm + qk == 27904
    assert bench.chain_bytes("bf16") == 27904 + 2048 == 29952
    assert bench.chain_bytes("q8") == 27904 + 512 + 32 + 512 == 28960
    assert bench.chain_bytes("q8_0") == bench.chain_bytes("q8_0_norot") == 27904 + 2 * 544
    assert bench.chain_bytes("bf16") * bench.TOKENS == 61341696


def test_hbm_bytes_from_request_counts():
    # a 32 MiB read: 262,144 requests of 128 bytes; a 32 MiB write: 524,288 of 64 bytes
    c = {"TCC_EA0_RDREQ_sum": 262144, "TCC_EA0_RDREQ_32B_sum": 0,
         "TCC_EA0_WRREQ_sum": 524288, "TCC_EA0_WRREQ_64B_sum": 524288}
    b = bench.hbm_bytes(c)
    assert b["read"] == b["write"] == 32 << 20 and b["total"] == 64 << 20
    # 32-byte requests count 32 bytes on both sides
    c = {"TCC_EA0_RDREQ_sum": 10, "TCC_EA0_RDREQ_32B_sum": 4,
         "TCC_EA0_WRREQ_sum": 10, "TCC_EA0_WRREQ_64B_sum": 6}
    b = bench.hbm_bytes(c)
    assert b["read"] == 6 * 128 + 4 * 32 and b["write"] == 6 * 64 + 4 * 32


def test_cold_sets():
    assert bench.cold_sets(61341696) == 25  # 1.5 GB / 61.3 MB, rounded up
    assert bench.cold_sets(490733568) == 4  # at least 4
    assert bench.cold_sets(490733568, least=1) == 4  # 1.5 GB / 490 MB, rounded up
    assert bench.cold_sets(2 * 10 ** 9, least=1) == 1
    for n in (4194304, 8388608, 20979712, 96542720, 132720640):
        assert bench.cold_sets(n) * n >= bench.COLD_BYTES


def test_copy_dispatch_filter():
    rows = [{"Kernel_Name": "k_stream_copy(a)", "Grid_Size": "119808"},
            {"Kernel_Name": "k_stream_copy(a)", "Grid_Size": "32768"},
            {"Kernel_Name": "k_chain<...>", "Grid_Size": "5120"},
            {"Kernel_Name": "k_stream_copy(a)", "Grid_Size_X": "120064"}]
    assert bench._largest_copy_grid(rows) == 120064
    assert bench._grid(rows[2]) == 5120 and bench._grid({"Kernel_Name": "x"}) is None


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_more_than_one_gpu_refused(gpus):
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", gpus],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stdout
