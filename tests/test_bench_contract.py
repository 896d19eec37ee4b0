"""bench.py's host-side pieces, without a GPU: the roofline objects, the HBM
traffic table it quotes (each line's bytes follow from its two counter
readings and the copy-kernel calibration, and no kernel moves fewer bytes than
its algorithmic figure), and the one-GPU guard of the command line."""
import os
import re
import subprocess
import sys

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LINE = re.compile(r"^(\w+): (\d+)\s+([\d.]+) ([\d.]+)\s+(\d+)\s+(.*)$")


def _rows():
    rows = {}
    with open(bench.TRAFFIC_FILE) as f:
        for line in f:
            if line.startswith("#") or not line.strip():
                continue
            m = LINE.match(line.rstrip("\n"))
            assert m, f"malformed traffic line: {line!r}"
            rows[m.group(1)] = m
    return rows


def test_traffic_table_lines_follow_from_the_counters():
    rows = _rows()
    # every key bench.py asks for is present
    for key in ("sgemm_4096", "conv2d", "mlp", "cnn", "skinny", "softmax", "eltwise_relu",
                "eltwise_add", "eltwise_mul", "copy"):
        assert key in rows, key
    for key, m in rows.items():
        total, fetch, write, algo = int(m.group(2)), float(m.group(3)), float(m.group(4)), \
            int(m.group(5))
        assert abs(total - (2.0 * fetch + 1.0 * write) * 1024) <= 1024, key
        # caches can only add traffic over the bytes the operator must move
        assert total >= 0.99 * algo, key
        tags = dict(f.split("=", 1) for f in m.group(6).split())
        assert re.fullmatch(r"[0-9a-f]{12}", tags["commit"]), key
        assert all(tags["kernels"].split(";")), key


def test_copy_calibration_reads_back_the_bytes_it_moved():
    m = _rows()["copy"]
    assert abs(int(m.group(2)) - 2 * 2**30) / 2**30 < 1e-4


def test_traffic_entry_parses_provenance():
    nbytes, src = bench._traffic_entry("skinny")
    assert nbytes == float(_rows()["skinny"].group(2))
    assert src["counters"] == "FETCH_SIZE, WRITE_SIZE"
    assert isinstance(src["kernels"], list) and len(src["kernels"]) == 2
    # template arguments keep their commas
    nbytes, src = bench._traffic_entry("conv2d")
    assert "sgemm_kernel<Tile<128,128,32,2,2,1,true>,0,5>" in src["kernels"]
    assert bench._traffic_entry("no_such_workload") == (None, None)


def test_roofline_objects():
    r = bench.roofline_mfma(157.3e9, 1.0)
    assert r == {"bound": "mfma", "achieved": 157.3, "peak": 157.3, "unit": "TFLOP/s",
                 "frac": 1.0, "traffic": None}
    r = bench.roofline_hbm(4e9, 1.0, "eltwise_relu")
    assert r["bound"] == "hbm" and r["achieved"] == 4000.0 and r["frac"] == 0.5
    assert r["traffic"] == float(_rows()["eltwise_relu"].group(2))
    assert r["traffic_source"]["kernels"] == ["relu_kernel"]


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(argv, env):
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *argv],
                         env={**os.environ, **env}, capture_output=True, text=True, timeout=300)
    assert out.returncode == 2
    assert "one GPU only" in out.stderr
    assert out.stdout == ""


CLINE = re.compile(r"^(\w+): ([\d.]+)\s+([\d.]+) ([\d.]+)\s+([\d.]+)\s+(.*)$")


def test_mfma_counter_table_parses_and_carries_provenance():
    rows = {}
    with open(bench.COUNTER_FILE) as f:
        for line in f:
            if line.startswith("#") or not line.strip():
                continue
            m = CLINE.match(line.rstrip("\n"))
            assert m, f"malformed counter line: {line!r}"
            rows[m.group(1)] = m
    # every MFMA-bound key bench.py asks for
    for key in ("sgemm_4096", "sgemm_2048", "sgemm_1024", "sgemm_8192", "mlp", "cnn", "conv2d"):
        assert key in rows, key
    for key, m in rows.items():
        busy, issued, algo, lds = (float(m.group(i)) for i in (2, 3, 4, 5))
        assert 0.0 < busy <= 1.0 and 0.0 <= lds < 1.0, key
        # the MFMA work issued is the algorithmic work up to padding, or less
        # where layers run outside the MFMAs (the CNN's conv1 and classifier)
        assert 0.9 * algo <= issued <= 1.1 * algo, key
        tags = dict(f.split("=", 1) for f in m.group(6).split())
        assert re.fullmatch(r"[0-9a-f]{12}", tags["commit"]), key
        assert all(tags["kernels"].split(";")), key
    busy, src = bench._counter_entry("sgemm_4096")
    assert busy == float(rows["sgemm_4096"].group(2))
    assert src["counters"] == "SQ_VALU_MFMA_BUSY_CYCLES, SQ_BUSY_CU_CYCLES"
    r = bench.roofline_mfma(137.4e9, 1.0, "sgemm_4096")
    assert r["mfma_busy"] == busy and r["mfma_busy_source"]["kernels"] == src["kernels"]
    # bandwidth rows carry no MFMA figure
    assert "mfma_busy" not in bench.roofline_hbm(4e9, 1.0, "eltwise_relu")
