"""bench.py --summarize on synthetic rocprofv3 CSV output (no GPU): dispatches are assigned to the
encoder's kernel classes by name and launch order (the residual GEMM is O after attention and wo
after the gated FFN), FETCH_SIZE / WRITE_SIZE are scaled by the copy calibration, and executed
MFMA work is read from SQ_INSTS_VALU_MFMA_MOPS_F16 (units of 512 FLOP, any instruction shape) or,
for the GEMMs only, from the instruction count of their 16x16x32 products."""
import csv
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

# one forward's launch order, with each dispatch's duration in ns
FORWARD = [
    ("embed_kernel(unsigned int const*, int)", 5000),
    ("void (anonymous namespace)::gemm_kernel<4, 0, 4, 128, 2, 0, false, 3>(GemmArgs, GemmGrid)", 20000),
    ("(anonymous namespace)::attn_relbias_kernel(AttnArgs)", 10000),
    ("void (anonymous namespace)::gemm_kernel<1, 0, 4, 64, 2, 0, false, 4>(GemmArgs, GemmGrid)", 16000),
    ("void (anonymous namespace)::gemm_kernel<2, 0, 4, 128, 2, 0, false, 3>(GemmArgs, GemmGrid)", 35000),
    ("void (anonymous namespace)::gemm_kernel<1, 0, 4, 64, 2, 0, false, 4>(GemmArgs, GemmGrid)", 26000),
    ("void (anonymous namespace)::gemm_kernel<3, 0, 2, 64, 2, 0, false, 4>(GemmArgs, GemmGrid)", 8000),
    ("(anonymous namespace)::rownorm_kernel(float*, float*, int, int, int, unsigned int*)", 4000),
]
CLASSES = ["embed_gather", "gemm_qkv", "attention", "gemm_o", "gemm_ffn_gate_up", "gemm_ffn_wo",
           "gemm_proj", "rownorm"]


def _write(path: Path, header, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def _trace(d: Path, forwards=2):
    rows, t, i = [], 1000, 1
    for _ in range(forwards):
        for name, ns in FORWARD:
            rows.append([i, name, t, t + ns])
            t += ns + 500
            i += 1
    _write(d / "kt_kernel_trace.csv", ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"], rows)


def _counters(d: Path, values, forwards=2):
    """values: class -> {counter: per-dispatch total}; each total is split over two instances, as
    per-XCD or per-SE rows are."""
    rows, i = [], 1
    for _ in range(forwards):
        for (name, _), c in zip(FORWARD, CLASSES):
            for counter, v in values.get(c, {}).items():
                rows.append([i, name, counter, v * 0.25])
                rows.append([i, name, counter, v * 0.75])
            i += 1
    _write(d / "b_counter_collection.csv", ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"], rows)


def _copy(d: Path, counter, kib):
    _write(d / "c_counter_collection.csv", ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"],
           [[1, "__amd_rocclr_copyBuffer", counter, kib]])


def _summarize(tmp: Path, counter_dirs):
    out = tmp / "traffic.json"
    cmd = [sys.executable, str(ROOT / "bench.py"), "--summarize", "--summarize-workload", "synthetic",
           "--trace", str(tmp / "kt"), "--counters", *map(str, counter_dirs),
           "--copy-fetch", str(tmp / "cfetch"), "--copy-write", str(tmp / "cwrite"),
           "--copy-bytes", str(1 << 20), "--out", str(out)]
    subprocess.run(cmd, check=True, cwd=ROOT, stdout=subprocess.DEVNULL)
    return json.loads(out.read_text())


def test_classes_durations_and_traffic(tmp_path):
    _trace(tmp_path / "kt")
    _copy(tmp_path / "cfetch", "FETCH_SIZE", 512.0)   # 1 MiB copied, read as 512 KiB: scale 2
    _copy(tmp_path / "cwrite", "WRITE_SIZE", 1024.0)  # scale 1
    _counters(tmp_path / "fetch", {c: {"FETCH_SIZE": 100.0 * (k + 1)} for k, c in enumerate(CLASSES)})
    _counters(tmp_path / "write", {c: {"WRITE_SIZE": 10.0 * (k + 1)} for k, c in enumerate(CLASSES)})
    d = _summarize(tmp_path, [tmp_path / "fetch", tmp_path / "write"])
    assert d["workload"] == "synthetic"
    assert abs(d["fetch_scale"] - 2.0) < 1e-12 and abs(d["write_scale"] - 1.0) < 1e-12
    for (name, ns), (k, c) in zip(FORWARD, enumerate(CLASSES)):
        assert abs(d["trace_avg_us"][c] - ns / 1000.0) < 1e-9, c
        b = d["bytes_per_dispatch"][c]
        assert abs(b["fetch"] - 100.0 * (k + 1) * 1024 * 2.0) < 1e-6, c
        assert abs(b["write"] - 10.0 * (k + 1) * 1024) < 1e-6, c
    # the two residual launches are told apart by what precedes them
    assert d["trace_avg_us"]["gemm_o"] == 16.0 and d["trace_avg_us"]["gemm_ffn_wo"] == 26.0


def test_mfma_work_from_mops_and_instruction_counts(tmp_path):
    _trace(tmp_path / "kt")
    _copy(tmp_path / "cfetch", "FETCH_SIZE", 512.0)
    _copy(tmp_path / "cwrite", "WRITE_SIZE", 1024.0)
    busy = {"SQ_VALU_MFMA_BUSY_CYCLES": 1024 * 100.0, "GRBM_GUI_ACTIVE": 8 * 400.0}  # 0.25 busy
    mops = {"attention": {"SQ_INSTS_VALU_MFMA_MOPS_F16": 3000.0, **busy},
            "gemm_qkv": {"SQ_INSTS_VALU_MFMA_MOPS_F16": 64.0, **busy}}
    _counters(tmp_path / "mops", mops)
    d = _summarize(tmp_path, [tmp_path / "mops"])
    assert d["counters"]["attention"]["mfma_flop_executed"] == 3000.0 * 512
    assert d["counters"]["gemm_qkv"]["mfma_flop_executed"] == 64.0 * 512
    assert abs(d["counters"]["gemm_qkv"]["mfma_busy_frac"] - 0.25) < 1e-12

    # instruction counts price the GEMMs' 16x16x32 products only; attention mixes shapes
    inst = {"attention": {"SQ_INSTS_VALU_MFMA_F16": 50.0, **busy},
            "gemm_o": {"SQ_INSTS_VALU_MFMA_F16": 50.0, **busy}}
    _counters(tmp_path / "inst", inst)
    d = _summarize(tmp_path, [tmp_path / "inst"])
    assert d["counters"]["gemm_o"]["mfma_flop_executed"] == 50.0 * 16 * 16 * 32 * 2
    assert "attention" not in d["counters"]
