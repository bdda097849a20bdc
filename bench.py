"""Benchmark of the MI355X ternary linear layer (one GPU).

Headline workload: the large-shape HBM stress at M=1 (K=8192 -> N=28672 and
K=28672 -> N=8192, fp16 scales |N(0,0.01)|, x ~ N(0,1)), each matrix in 8
rotating device copies (about 500 MB, more than the 256 MB Infinity Cache),
so every call streams its weights from HBM.  One step is one cold GEMV of
each shape through the reference-named entry point ``gemv_plain_store``
(quantize + GEMV).  W warmup steps run untimed; then exactly K steps are
recorded into one HIP graph, which is replayed 20 times with events on the
launch stream around each replay: ``ms_per_step`` is the median replay / K.
``value`` is algorithmic bytes / second over the timed steps:
bytes(M,N,K) = N*ceil(K/4) + 2*N*ceil(K/128) + 4*M*K + 4*M*N.

Also reported on the same line: the roofline figure of the kernel the
headline times (the launch gemv_plain_store makes, quantizing the row in
every block), from the dispatch durations of a rocprofv3 kernel-trace pass
the bench runs itself, with the HIP-event time per call inside a graph of 8
back-to-back calls beside it, and the same figures for the GEMV alone on
pre-quantized activations (`roofline.prequant`); the
single-linear case (K=1024 -> N=4096), the 32-token prefill tile GEMM TOPS,
and the CPU baseline (the reference's numba GEMV restated in C++/OpenMP)
on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "ivonar-inference_amd"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
ROTATING_COPIES = 8
HEADLINE_REPLAYS = 20
PROBE_GEMM_SHAPES = [(1024, 4096), (4096, 1024), (4096, 14336)]  # (K, N) of the GEMM probe, in order
PROBE_GEMM_M = (2048, 32)
PROBE_BIG_READ_BYTES = 1 << 30
PROBE_BIG_READS = 4


def gemv_bytes(m: int, n: int, k: int) -> int:
    return n * ((k + 3) // 4) + 2 * n * ((k + 127) // 128) + 4 * m * k + 4 * m * n


def parse() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU-baseline sample")
    parser.add_argument("--skip-cpu", action="store_true")
    parser.add_argument("--probe", choices=["gemv-stress", "gemm-prefill", "tokens"], default=None,
                        help="profiling mode: only the named kernel workload, no JSON line")
    parser.add_argument("--probe-calls", type=int, default=16)
    parser.add_argument("--no-traffic", action="store_true", help="skip the three rocprofv3 counter passes")
    return parser.parse_args()


def probe_gemv_stress(calls: int) -> None:
    """On both stress shapes, cycling 8 copies: `calls` launches of gemv_plain_store (the launch quantizes
    the fp32 row itself: the kernel the headline times), then `calls` launches of the GEMV on
    pre-quantized input, then the streaming-read kernel once over each copy's packed bytes (58.7 MB
    launches); then PROBE_BIG_READS streaming reads of one 1 GiB buffer; then a 512 MiB device copy of
    known size that calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    from ivonar_amd import ops, runtime, synthetic

    device = torch.device("cuda", 0)
    runtime.initialise(0)
    lib = runtime.library()
    sink = torch.empty(lib.ivonar_stream_read_sink_words(), dtype=torch.int32, device=device)
    stream_id = runtime.current_stream()

    def stream_read(tensor):
        runtime.check(lib.ivonar_stream_read(stream_id, runtime.pointer(tensor), tensor.numel(), runtime.pointer(sink)),
                      "ivonar_stream_read")

    for layer, x in synthetic.stress_layers(seed=3):
        mats = device_copies(layer, device, ROTATING_COPIES)
        xd = torch.from_numpy(x).to(device)
        q8, xsum, sx = ops.quantize_rows(xd)
        out = torch.empty(layer.rows, dtype=torch.float32, device=device)
        torch.cuda.synchronize()
        for call in range(calls):
            ops.gemv(mats[call % ROTATING_COPIES], xd[0], out=out)
        torch.cuda.synchronize()
        for call in range(calls):
            ops.gemv_prequant(mats[call % ROTATING_COPIES], q8, xsum, sx, out=out)
        torch.cuda.synchronize()
        for mat in mats:
            stream_read(mat.packed)
        torch.cuda.synchronize()
        print(f"probe: gemv {layer.in_features}->{layer.rows} x{calls}, {len(mats)} reads done", flush=True)
        del mats
    big = torch.empty(PROBE_BIG_READ_BYTES, dtype=torch.uint8, device=device)  # contents unused: no fill dispatch
    torch.cuda.synchronize()
    for _ in range(PROBE_BIG_READS):
        stream_read(big)
    torch.cuda.synchronize()
    del big
    print(f"probe: {PROBE_BIG_READS} reads of 1 GiB done", flush=True)
    src = torch.empty(512 * 2**20, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    print("probe: 512 MiB copy done", flush=True)


def probe_tokens(calls: int) -> None:
    """GEMM with M = 1, 2, 4, 8, 16 tokens on both stress shapes (pre-quantized activations), `calls`
    launches per M cycling the 8 rotating copies: the token GEMV, or the skinny kernel where the tokens'
    q8 rows do not fit in LDS."""
    import numpy as np
    import torch

    from ivonar_amd import ops, runtime, synthetic

    device = torch.device("cuda", 0)
    runtime.initialise(0)
    rng = np.random.default_rng(11)
    for layer, _ in synthetic.stress_layers(seed=3):
        mats = device_copies(layer, device, ROTATING_COPIES)
        for m in (1, 2, 4, 8, 16):
            x = torch.from_numpy(rng.standard_normal((m, layer.in_features)).astype(np.float32)).to(device)
            q8, xsum, sx = ops.quantize_rows(x)
            out = torch.empty((m, layer.rows), dtype=torch.float32, device=device)
            torch.cuda.synchronize()
            for call in range(calls):
                ops.gemm(mats[call % ROTATING_COPIES], q8, xsum, sx, out=out)
            torch.cuda.synchronize()
            print(f"probe: tokens m={m} {layer.in_features}->{layer.rows} x{calls} done", flush=True)
        del mats


def probe_gemm_prefill(calls: int) -> None:
    """Token GEMM alone at M=2048 and M=32 on both prefill shapes and on K=4096 -> N=14336
    (pre-quantized activations)."""
    import numpy as np
    import torch

    from ivonar_amd import ops, runtime, synthetic

    device = torch.device("cuda", 0)
    runtime.initialise(0)
    props = torch.cuda.get_device_properties(device)
    print(f"probe: {props.name} CUs={props.multi_processor_count} "
          f"lds_per_block={getattr(props, 'shared_memory_per_block', '?')}", flush=True)
    rng = np.random.default_rng(2)
    sweep, _ = synthetic.sweep_layer(seed=4)
    layers = [*synthetic.prefill_layers(seed=2), (sweep, sweep.in_features)]
    if [(k, layer.rows) for layer, k in layers] != PROBE_GEMM_SHAPES:
        raise RuntimeError("GEMM probe shapes changed")
    for layer, k in layers:
        mat = device_copies(layer, device, 1)[0]
        for m in PROBE_GEMM_M:
            xs = torch.from_numpy(synthetic.prefill_activations(rng, m, k)).to(device)
            q8, xsum, sx = ops.quantize_rows(xs)
            out = torch.empty((m, layer.rows), dtype=torch.float32, device=device)
            torch.cuda.synchronize()
            for _ in range(calls):
                ops.gemm(mat, q8, xsum, sx, out=out)
            torch.cuda.synchronize()
            print(f"probe: gemm m={m} {k}->{layer.rows} x{calls} done", flush=True)


def graph_of(step, stream):
    import torch

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    return graph


def time_graph(graph, replays: int, warmup: int, median: bool = False) -> float:
    """Seconds per replay on the current stream: HIP events around all `replays` replays (the mean), or
    with `median`, around each replay and the median of those."""
    import torch

    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    if median:
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
        marks[0].record()
        for index in range(replays):
            graph.replay()
            marks[index + 1].record()
        torch.cuda.synchronize()
        times = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(replays))
        return times[len(times) // 2] / 1e3
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / replays


def copy_bandwidth(device, stream, size: int = 1 << 30) -> dict:
    """Device-to-device copy of `size` bytes (torch's copy kernel), 4 copies per HIP graph, median of 20
    replays; bandwidth counts the bytes read plus the bytes written."""
    import torch

    src = torch.empty(size, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    src.fill_(1)
    graph = graph_of(lambda: [dst.copy_(src) for _ in range(4)], stream)
    seconds = time_graph(graph, 20, 2, median=True) / 4
    del src, dst
    return {"GBps": round(2 * size / seconds / 1e9, 1), "bytes_moved": 2 * size, "us": round(seconds * 1e6, 2)}


def read_ceiling(matrices, stream) -> dict:
    """Streaming-read bandwidth over the packed weights the GEMV streams (8 rotating copies of both stress
    matrices, 58.7 MB each), one launch per matrix, timed like the GEMV: the best a kernel that only reads
    achieves per launch at this size; and the same kernel over one 1 GiB buffer in one launch (the sustained
    rate, without the per-launch ramp and drain)."""
    import torch

    from ivonar_amd import runtime

    lib = runtime.library()
    device = matrices[0][0].packed.device
    sink = torch.empty(lib.ivonar_stream_read_sink_words(), dtype=torch.int32, device=device)
    buffers = [(m.packed, m.packed.numel()) for shape in matrices for m in shape]
    total = sum(size for _, size in buffers)

    def read(items):
        def run():
            stream_id = runtime.current_stream()
            for tensor, size in items:
                runtime.check(lib.ivonar_stream_read(stream_id, runtime.pointer(tensor), size, runtime.pointer(sink)),
                              "ivonar_stream_read")
        return run

    seconds = time_graph(graph_of(read(buffers), stream), 20, 2, median=True)
    big = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    big.fill_(1)
    big_seconds = time_graph(graph_of(read([(big, big.numel())]), stream), 20, 2, median=True)
    del big
    return {"GBps": round(total / seconds / 1e9, 1), "bytes": total, "us_per_launch": round(seconds / len(buffers) * 1e6, 3),
            "one_GiB_launch": {"GBps": round((1 << 30) / big_seconds / 1e9, 1), "us": round(big_seconds * 1e6, 2)},
            "kernel": "ivonar_stream_read (non-temporal 16-byte loads, 4 in flight per thread, 1024 blocks)"}


def validate_throughput(matrices, stream) -> dict:
    """ivonar_validate_ternary (the checkpoint loader's device check: reserved codes, non-finite or
    non-positive scales) over the 16 stress operands, one launch each, median of 20 graph replays."""
    from ivonar_amd import checkpoint

    operands = [m for shape in matrices for m in shape]
    total = sum(m.packed.numel() + 2 * m.scales.numel() for m in operands)

    def run():
        for m in operands:
            checkpoint.validation_flags(m.packed, m.scales)

    seconds = time_graph(graph_of(run, stream), 20, 2, median=True)
    return {"GBps": round(total / seconds / 1e9, 1), "bytes": total, "us_per_operand": round(seconds / len(operands) * 1e6, 2)}


def time_calls(call, stream, calls_per_graph: int, replays: int, warmup: int = 2, warm_ms: float = 0.0) -> float:
    """Seconds per call: `calls_per_graph` back-to-back calls recorded in one HIP graph, so that the time of
    a short kernel is not the host's graph-launch time.  With `warm_ms`, the graph is first replayed for about
    that long (sustained MFMA work runs slower for its first ~20 ms on a fresh box)."""
    graph = graph_of(lambda: [call() for _ in range(calls_per_graph)], stream)
    if warm_ms > 0:
        estimate = time_graph(graph, 2, 1)
        warmup = max(warmup, int(warm_ms * 1e-3 / max(estimate, 1e-6)) + 1)
    return time_graph(graph, replays, warmup) / calls_per_graph


def device_copies(layer, device, copies: int):
    import torch
    from ivonar_amd.matrix import Matrix

    base = Matrix.from_tensors(torch.from_numpy(layer.packed), torch.from_numpy(layer.scales), layer.in_features,
                               device=device)
    mats = [base]
    for _ in range(copies - 1):
        clone = Matrix.__new__(Matrix)
        for slot in Matrix.__slots__:
            setattr(clone, slot, getattr(base, slot))
        clone.packed = base.packed.clone()
        clone.scales = base.scales.clone()
        mats.append(clone)
    return mats


def counter_pass(counters: list[str], probe: str, calls: int) -> list[dict] | str:
    """One rocprofv3 counter pass over `bench.py --probe <probe>` as a child process (this process has not
    touched the GPU yet): the per-dispatch rows of its counter CSV, or an error string."""
    import csv
    import shutil
    import subprocess
    import tempfile

    tool = shutil.which("rocprofv3")
    if tool is None:
        return "rocprofv3 not found"
    out = tempfile.mkdtemp(prefix="ivonar_pmc_", dir="/tmp")
    command = [tool, "--pmc", *counters, "--output-format", "csv", "-d", out, "-o", "pmc", "--",
               sys.executable, str(ROOT / "bench.py"), "--probe", probe, "--probe-calls", str(calls)]
    print(f"bench: counter pass {' '.join(counters)} over {probe}", file=sys.stderr, flush=True)
    try:
        done = subprocess.run(command, cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"}, timeout=240,
                              stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    except subprocess.TimeoutExpired:
        shutil.rmtree(out, ignore_errors=True)
        return f"{counters} pass timed out"
    files = sorted(Path(out).rglob("*counter_collection.csv"))
    if not files:
        shutil.rmtree(out, ignore_errors=True)
        return f"{counters} pass exited {done.returncode} without a counter file: {done.stdout[-300:]}"
    dispatches: dict[int, dict] = {}
    with open(files[0]) as handle:
        for row in csv.DictReader(handle):
            entry = dispatches.setdefault(int(row["Dispatch_Id"]), {"kernel": row["Kernel_Name"],
                                                                   "grid": int(row["Grid_Size"])})
            entry[row["Counter_Name"]] = entry.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    shutil.rmtree(out, ignore_errors=True)
    return [dispatches[key] for key in sorted(dispatches)]


def measure_traffic(calls: int = 8) -> dict:
    """HBM bytes per GEMV dispatch from two counter passes (FETCH_SIZE, then WRITE_SIZE) over the GEMV
    probe, each scaled by what the counter reads for the probe's 512 MiB device copy."""
    readings: dict[str, dict] = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        rows = counter_pass([counter], "gemv-stress", calls)
        if isinstance(rows, str):
            return {"error": rows}
        gemv, reads, other = {}, [], []
        for row in rows:
            if counter not in row:
                continue
            if "gemv_kernel" in row["kernel"] or "gemv_rows_kernel" in row["kernel"]:
                gemv.setdefault((_short_name(row["kernel"]), row["grid"]), []).append(row[counter])
            elif "stream_read" in row["kernel"]:
                reads.append(row[counter])
            else:
                other.append(row[counter])
        if not gemv or not other:
            return {"error": f"{counter} pass found no GEMV or copy dispatch"}
        readings[counter] = {"factor": (512 * 1024) / max(other),
                             "per_grid": {grid: sum(v) / len(v) for grid, v in gemv.items()}, "reads": reads}
    fetch, write = readings["FETCH_SIZE"], readings["WRITE_SIZE"]
    launch_bytes = {key: fetch["per_grid"][key] * fetch["factor"] * 1024 + write["per_grid"].get(key, 0.0) * write["factor"] * 1024
                    for key in fetch["per_grid"]}
    # the quantizing kernels (QUANT true: the kernel the headline times) and the pre-quantized ones
    per_launch = [v for (name, _), v in launch_bytes.items() if _quantizing(name)]
    prequant_launch = [v for (name, _), v in launch_bytes.items() if not _quantizing(name)]
    # streaming-read launches: the last PROBE_BIG_READS read the 1 GiB buffer, the others one packed copy each
    reads = [v * fetch["factor"] * 1024 for v in fetch["reads"]]
    read_fetch = None
    if len(reads) > PROBE_BIG_READS:
        small, big = reads[:-PROBE_BIG_READS], reads[-PROBE_BIG_READS:]
        read_fetch = {"copy_launch_bytes": round(sum(small) / len(small)), "one_GiB_launch_bytes": round(sum(big) / len(big)),
                      "note": "FETCH_SIZE x factor per streaming-read dispatch: 58.7 MB packed-copy launches and "
                              "1 GiB launches (1,073,741,824 bytes read)"}
    if not per_launch or not prequant_launch:
        return {"error": "the counter passes did not find both the quantizing and the pre-quantized GEMV"}
    return {"bytes_per_launch": sum(per_launch) / len(per_launch),
            "fetch_factor": round(fetch["factor"], 4), "write_factor": round(write["factor"], 4),
            "per_launch": {f"{name} [{grid}]": round(v) for (name, grid), v in launch_bytes.items()},
            "prequant_bytes_per_launch": sum(prequant_launch) / len(prequant_launch),
            "stream_read_fetch": read_fetch}


def _short_name(kernel: str) -> str:
    """`gemv_rows_kernel<0, 7, true, true, 1>` from a demangled kernel name (template kernels carry a `void `
    return type in the trace, the others do not)."""
    name = kernel.strip()
    if name.startswith("void "):
        name = name[len("void "):]
    return name.replace("ivo::(anonymous namespace)::", "").split("(")[0].strip()


def _quantizing(name: str) -> bool:
    """Whether a `gemv_rows_kernel<EPI, STEPS, EXACT, QUANT, TOKENS>` name is the quantizing launch (QUANT true)."""
    if "<" not in name or ">" not in name:
        return False
    args = [a.strip() for a in name[name.index("<") + 1:name.rindex(">")].split(",")]
    return len(args) >= 4 and args[3] == "true"


def measure_trace(calls: int = 32) -> dict:
    """Dispatch durations of the GEMV kernels alone: one `rocprofv3 --kernel-trace --stats` pass over the GEMV
    probe (pre-quantized input, `calls` launches per stress shape cycling the 8 copies), as a child process;
    the average duration per kernel and the bandwidth it implies for one stress GEMV."""
    import csv
    import shutil
    import subprocess
    import tempfile

    tool = shutil.which("rocprofv3")
    if tool is None:
        return {"error": "rocprofv3 not found"}
    out = tempfile.mkdtemp(prefix="ivonar_trace_", dir="/tmp")
    command = [tool, "--kernel-trace", "--stats", "--output-format", "csv", "-d", out, "-o", "trace", "--",
               sys.executable, str(ROOT / "bench.py"), "--probe", "gemv-stress", "--probe-calls", str(calls)]
    print("bench: kernel-trace pass over gemv-stress", file=sys.stderr, flush=True)
    try:
        subprocess.run(command, cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"}, timeout=240,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    except subprocess.TimeoutExpired:
        shutil.rmtree(out, ignore_errors=True)
        return {"error": "kernel-trace pass timed out"}
    files = sorted(Path(out).rglob("*kernel_stats.csv"))
    if not files:
        shutil.rmtree(out, ignore_errors=True)
        return {"error": "kernel-trace pass wrote no kernel_stats.csv"}
    kernels = {}
    with open(files[0]) as handle:
        reader = csv.DictReader(handle)
        if not {"Name", "Calls", "AverageNs"} <= set(reader.fieldnames or []):
            shutil.rmtree(out, ignore_errors=True)
            return {"error": f"unexpected kernel_stats.csv columns {reader.fieldnames}"}
        for row in reader:
            if "gemv" in row["Name"]:
                kernels[_short_name(row["Name"])] = {"calls": int(row["Calls"]),
                                                     "average_us": round(float(row["AverageNs"]) / 1e3, 3)}
    # streaming reads, per dispatch in launch order: one per packed copy of each shape, then the 1 GiB reads
    reads = []
    for path in sorted(Path(out).rglob("*kernel_trace.csv")):
        with open(path) as handle:
            reader = csv.DictReader(handle)
            if not {"Kernel_Name", "Start_Timestamp", "End_Timestamp"} <= set(reader.fieldnames or []):
                continue
            rows = [row for row in reader if "stream_read" in row["Kernel_Name"]]
        rows.sort(key=lambda row: int(row["Start_Timestamp"]))
        reads = [(int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3 for row in rows]
    shutil.rmtree(out, ignore_errors=True)
    per_launch = 62537728
    result = {"kernels": kernels,
              "GBps_from_average": {k: round(per_launch / (v["average_us"] * 1e3), 1) for k, v in kernels.items()},
              "note": "dispatch durations from the trace exclude the gap between back-to-back launches"}
    if len(reads) == 2 * ROTATING_COPIES + PROBE_BIG_READS:
        small, big = reads[:2 * ROTATING_COPIES], reads[2 * ROTATING_COPIES:]
        copy_bytes = 28672 * 8192 // 4  # the packed bytes of either stress shape: 58,720,256
        result["stream_read"] = {
            "copy_launch_us": round(sum(small) / len(small), 3),
            "copy_launch_GBps": round(copy_bytes / (sum(small) / len(small) * 1e3), 1),
            "one_GiB_launch_us": round(sum(big) / len(big), 2),
            "one_GiB_launch_GBps": round(PROBE_BIG_READ_BYTES / (sum(big) / len(big) * 1e3), 1)}
    else:
        result["stream_read"] = {"error": f"expected {2 * ROTATING_COPIES + PROBE_BIG_READS} streaming-read dispatches, "
                                          f"found {len(reads)}"}
    return result


def measure_mfma(calls: int = 16, cus: int = 256, xcds: int = 8) -> dict:
    """MFMA-busy share of the token GEMM from one counter pass over the GEMM probe, per case: rocprofv3's
    derived MfmaUtil (SQ_VALU_MFMA_BUSY_CYCLES summed over SIMDs / (GRBM_GUI_ACTIVE max over XCDs x SIMDs)),
    the same ratio from the raw counters (GRBM_GUI_ACTIVE as read is the sum over the XCDs), and the int8
    ops the MFMA unit counted (SQ_INSTS_VALU_MFMA_MOPS_I8 x 512) against 2*M*N*K."""
    counters = ["MfmaUtil", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_I8", "GRBM_GUI_ACTIVE"]
    rows = counter_pass(counters, "gemm-prefill", calls)
    if isinstance(rows, str):
        return {"error": rows}
    kernels = ("gemm_kernel", "gemm_wide_kernel", "gemm_split_kernel", "skinny_kernel", "skinny_row_kernel")
    gemm = [row for row in rows if any(name in row["kernel"] for name in kernels) and all(c in row for c in counters)]
    cases = [(k, n, m) for k, n in PROBE_GEMM_SHAPES for m in PROBE_GEMM_M]
    if len(gemm) != len(cases) * calls:
        return {"error": f"expected {len(cases) * calls} GEMM dispatches, found {len(gemm)}"}
    table = {}
    for index, (k, n, m) in enumerate(cases):
        chunk = gemm[index * calls:(index + 1) * calls]

        def mean(name, chunk=chunk):
            return sum(r[name] for r in chunk) / calls

        busy, active = mean("SQ_VALU_MFMA_BUSY_CYCLES"), mean("GRBM_GUI_ACTIVE")
        name = chunk[0]["kernel"].replace("void ivo::(anonymous namespace)::", "").split("(")[0]
        table[f"{k}x{n}_M{m}"] = {"MfmaUtil_pct": round(mean("MfmaUtil"), 2),
                                  "busy_share_raw": round(busy * xcds / (active * 4 * cus), 4),
                                  "mfma_ops_counted": int(mean("SQ_INSTS_VALU_MFMA_MOPS_I8") * 512),
                                  "ops_algorithmic": 2 * m * n * k, "kernel": name}
    return {"by_case": table, "simds": 4 * cus,
            "note": "GRBM_GUI_ACTIVE covers the whole dispatch under counter collection, launch and drain included"}


def m_sweep(device, stream) -> dict:
    """K=4096 -> N=14336 with p(0)=0.6, lognormal(-4, 0.5) scales and Student-t(3) activations: the GEMV
    (one launch per token) against the token GEMM for M in 1..2048, weights warm in the caches."""
    import torch

    from ivonar_amd import ops, synthetic

    layer, rng = synthetic.sweep_layer(seed=4)
    mat = device_copies(layer, device, 1)[0]
    k, n = layer.in_features, layer.rows
    table = {}
    crossover = None
    for m in synthetic.SWEEP_M:
        x = torch.from_numpy(synthetic.student_t(rng, (m, k))).to(device)
        q8, xsum, sx = ops.quantize_rows(x)
        out = torch.empty((m, n), dtype=torch.float32, device=device)
        # Long prompts: about 25 ms of the same calls before the timed replays (the first 20 ms of
        # sustained MFMA load on a fresh box run up to 20% slower than the steady state).
        t_gemm = time_calls(lambda: ops.gemm(mat, q8, xsum, sx, out=out), stream, 20 if m <= 128 else 4, 10,
                            warm_ms=25.0 if m >= 512 else 0.0)
        entry = {"gemm_us": round(t_gemm * 1e6, 3), "gemm_TOPS": round(2 * m * n * k / t_gemm / 1e12, 2)}
        if m <= 16:
            rows = [(q8[i], xsum[i], sx[i:i + 1], out[i]) for i in range(m)]

            def per_token(rows=rows):
                for q, xs, s, o in rows:
                    ops.gemv_prequant(mat, q, xs, s, out=o)

            t_gemv = time_calls(per_token, stream, 10, 10)
            entry["gemv_us"] = round(t_gemv * 1e6, 3)
            if crossover is None and t_gemm < t_gemv:
                crossover = m
        table[str(m)] = entry
    return {"shape": f"{k}x{n}", "by_m": table, "gemm_faster_from_m": crossover,
            "note": "weights warm in the caches; 20 (M <= 128) or 4 calls per HIP graph, M >= 512 after 25 ms "
                    "of the same calls; gemm_us for M = 1 is the decode GEMV on the pre-quantized row, for "
                    "M = 2 the two-token GEMV on rows of 4097..32768 inputs, else for M = 2..16 the token GEMV "
                    "(K a multiple of 256)"}


def stress_tokens(matrices, stress, stream, replays: int) -> dict:
    """Cold-cache GEMM with M = 1..16 tokens on the two stress shapes (8 rotating copies per shape, one
    HIP graph of 8 calls, median of `replays` replays): M = 1 runs the decode GEMV and M = 2 the two-token
    GEMV (plan 0), M = 4..16 the token GEMV (plan = its K-splits); beside it the M = 1 GEMV on pre-quantized
    input called directly."""
    import numpy as np
    import torch

    from ivonar_amd import ops, runtime

    rng = np.random.default_rng(11)
    table = {}
    for shape, (layer, _) in enumerate(stress):
        k, n = layer.in_features, layer.rows
        out = torch.empty((16, n), dtype=torch.float32, device=matrices[shape][0].packed.device)
        entry = {}
        for m in (1, 2, 4, 8, 16):
            x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(out.device)
            q8, xsum, sx = ops.quantize_rows(x)

            def run(q8=q8, xsum=xsum, sx=sx, m=m):
                for mat in matrices[shape]:
                    ops.gemm(mat, q8, xsum, sx, out=out[:m])

            t = time_graph(graph_of(run, stream), replays, 2, median=True) / len(matrices[shape])
            entry[str(m)] = {"us": round(t * 1e6, 3), "GBps": round(gemv_bytes(m, n, k) / t / 1e9, 1),
                             "plan": runtime.gemm_plan(m, n, k)}
        q8, xsum, sx = ops.quantize_rows(torch.from_numpy(rng.standard_normal((1, k)).astype(np.float32)).to(out.device))

        def gemv(q8=q8, xsum=xsum, sx=sx):
            for mat in matrices[shape]:
                ops.gemv_prequant(mat, q8, xsum, sx, out=out[0])

        t1 = time_graph(graph_of(gemv, stream), replays, 2, median=True) / len(matrices[shape])
        entry["gemv_m1_us"] = round(t1 * 1e6, 3)
        entry["m16_over_gemv_m1"] = round(entry["16"]["us"] / entry["gemv_m1_us"], 3)
        entry["m16_over_m1"] = round(entry["16"]["us"] / entry["1"]["us"], 3)
        entry["m2_over_gemv_m1"] = round(entry["2"]["us"] / entry["gemv_m1_us"], 3)
        table[f"{k}x{n}"] = entry
    return {"by_shape": table, "timing": "median of HIP-graph replays of 8 calls (one per rotating copy), per call"}


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; multi-GPU figures are not part of this build",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.probe == "gemv-stress":
        probe_gemv_stress(args.probe_calls)
        return
    if args.probe == "gemm-prefill":
        probe_gemm_prefill(args.probe_calls)
        return
    if args.probe == "tokens":
        probe_tokens(args.probe_calls)
        return
    import numpy as np
    import torch

    from ivonar_amd import ops, runtime, synthetic

    traffic = None if args.no_traffic else measure_traffic()
    trace = None if args.no_traffic else measure_trace()
    mfma = None if args.no_traffic else measure_mfma()
    device = torch.device("cuda", 0)
    runtime.initialise(0)
    stream = torch.cuda.Stream()
    results: dict[str, object] = {}

    # ---- headline: cold-cache GEMV at the stress shapes -------------------------------------
    stress = synthetic.stress_layers(seed=3)
    matrices, inputs, outputs, bytes_per_step = [], [], [], 0
    for layer, x in stress:
        matrices.append(device_copies(layer, device, ROTATING_COPIES))
        inputs.append(torch.from_numpy(x[0]).to(device))
        outputs.append(torch.empty(layer.rows, dtype=torch.float32, device=device))
        bytes_per_step += gemv_bytes(1, layer.rows, layer.in_features)

    def stress_steps(count: int, first: int = 0):
        def run():
            for step in range(first, first + count):
                copy = step % ROTATING_COPIES
                for shape in range(len(stress)):
                    ops.gemv(matrices[shape][copy], inputs[shape], out=outputs[shape])
        return run

    # W untimed warmup steps, then HEADLINE_REPLAYS replays of one HIP graph of exactly K steps, each
    # replay bracketed by events on the launch stream; the median replay is the timed K steps.
    steps = args.steps
    with torch.cuda.stream(stream):
        stress_steps(args.warmup)()
    torch.cuda.synchronize()
    graph = graph_of(stress_steps(steps), stream)
    seconds = time_graph(graph, HEADLINE_REPLAYS, 1, median=True)
    step_seconds = seconds / steps
    value = bytes_per_step / step_seconds / 1e9

    # ---- the kernels per shape: the headline's (quantize + GEMV in one launch) and the GEMV alone on
    # pre-quantized activations.  Per call inside a HIP graph of 8 back-to-back calls (one per rotating
    # copy), events on the launch stream around each replay; the inter-launch gap a decode sequence also
    # pays is included.  The kernel-trace pass below gives the dispatch durations alone.
    kernel, prequant_kernel = {}, {}
    replays = max(20, args.steps // ROTATING_COPIES)
    for shape, (layer, x) in enumerate(stress):
        q8, xsum, sx = ops.quantize_rows(inputs[shape].reshape(1, -1))
        b = gemv_bytes(1, layer.rows, layer.in_features)

        def plain(shape=shape):
            for copy in range(ROTATING_COPIES):
                ops.gemv(matrices[shape][copy], inputs[shape], out=outputs[shape])

        def prequant(shape=shape, q8=q8, xsum=xsum, sx=sx):
            for copy in range(ROTATING_COPIES):
                ops.gemv_prequant(matrices[shape][copy], q8, xsum, sx, out=outputs[shape])

        name = f"{layer.in_features}x{layer.rows}"
        t = time_graph(graph_of(plain, stream), replays, 2, median=True) / ROTATING_COPIES
        kernel[name] = {"us": t * 1e6, "GBps": b / t / 1e9, "bytes": b}
        t = time_graph(graph_of(prequant, stream), replays, 2, median=True) / ROTATING_COPIES
        prequant_kernel[name] = {"us": t * 1e6, "GBps": b / t / 1e9, "bytes": b}
    # the same shapes with 1..16 tokens through the gemm_tile_store path (token GEMV / skinny kernel)
    results["stress_tokens"] = stress_tokens(matrices, stress, stream, max(20, args.steps // ROTATING_COPIES))
    kernel_bytes = sum(v["bytes"] for v in kernel.values())

    def graph_rate(per_shape: dict) -> float:
        return kernel_bytes / (sum(v["us"] for v in per_shape.values()) / 1e6) / 1e9

    def trace_rate(quant: bool):
        """Algorithmic bytes per launch over the mean dispatch duration of the quantizing (or the
        pre-quantized) GEMV kernels in the kernel-trace pass, or None."""
        if not trace or not trace.get("kernels"):
            return None
        chosen = {k: v for k, v in trace["kernels"].items() if _quantizing(k) == quant}
        if not chosen:
            return None
        calls = sum(v["calls"] for v in chosen.values())
        mean_us = sum(v["calls"] * v["average_us"] for v in chosen.values()) / calls
        return (kernel_bytes / len(kernel)) / (mean_us * 1e-6) / 1e9

    achieved_graph, prequant_graph = graph_rate(kernel), graph_rate(prequant_kernel)
    achieved, prequant_achieved = trace_rate(True), trace_rate(False)
    timing = ("algorithmic bytes per launch / mean dispatch duration of the quantizing GEMV kernels "
              "(gemv_rows_kernel<..., true>, what gemv_plain_store launches) in the rocprofv3 kernel-trace pass "
              "(kernel_trace); achieved_graph is the HIP-event time per call inside a graph of 8 back-to-back "
              "calls, median of >= 20 replays, inter-launch gaps included")
    if achieved is None:
        achieved, prequant_achieved = achieved_graph, prequant_graph
        timing = ("algorithmic bytes / time per call: median of >= 20 replays of a HIP graph of 8 back-to-back calls "
                  "(one per rotating copy), events on the launch stream, inter-launch gaps included (the "
                  "kernel-trace pass failed)")
    ceiling = read_ceiling(matrices, stream)
    results["checkpoint_validate"] = validate_throughput(matrices, stream)
    copy = copy_bandwidth(device, stream)

    # ---- single linear K=1024 -> N=4096 (launch-latency bound) ------------------------------
    layer0, x0 = synthetic.single_linear(seed=0)
    m0 = device_copies(layer0, device, 1)[0]
    xin0 = torch.from_numpy(x0[0]).to(device)
    y0 = torch.empty(layer0.rows, dtype=torch.float32, device=device)
    g0 = graph_of(lambda: [ops.gemv(m0, xin0, out=y0) for _ in range(64)], stream)
    t0 = time_graph(g0, 20, 2) / 64
    results["single_linear_1024x4096_us"] = round(t0 * 1e6, 3)

    # ---- prefill GEMM: prompts of L tokens as 32-token tiles and as one launch ----------------------
    rng = np.random.default_rng(2)
    prefill = {}
    for layer, k in synthetic.prefill_layers(seed=2):
        mat = device_copies(layer, device, 1)[0]
        shape = {}
        for length in (32, 128, 512, 2048):
            xs = torch.from_numpy(synthetic.prefill_activations(rng, length, k)).to(device)
            q8, xsum, sx = ops.quantize_rows(xs)
            out = torch.empty((length, layer.rows), dtype=torch.float32, device=device)
            tiles = [(q8[t:t + 32], xsum[t:t + 32], sx[t:t + 32], out[t:t + 32]) for t in range(0, length, 32)]

            def tiled(tiles=tiles):
                for q, x, s_, o in tiles:
                    ops.gemm(mat, q, x, s_, out=o)

            t_tiles = time_calls(tiled, stream, max(1, 64 // len(tiles)), 10)
            t_one = time_calls(lambda: ops.gemm(mat, q8, xsum, sx, out=out), stream, 20 if length <= 128 else 4, 10,
                               warm_ms=25.0 if length >= 512 else 0.0)
            ops_count = 2 * length * layer.rows * k
            shape[str(length)] = {"tiles_us": round(t_tiles * 1e6, 3), "tiles_TOPS": round(ops_count / t_tiles / 1e12, 2),
                                  "one_launch_us": round(t_one * 1e6, 3),
                                  "one_launch_TOPS": round(ops_count / t_one / 1e12, 2)}
        prefill[f"{k}x{layer.rows}"] = shape
    results["prefill_gemm"] = prefill
    results["prefill_gemm_counters"] = mfma

    # ---- decoder-shaped stack: greedy decode tok/s, and the device sampler -------------------------
    results["decode_stack"] = decode_stack(device)
    results["decode_stack_sampled"] = decode_stack(device, sampling=(0.8, 40, 1.1))
    results["sampler"] = sampler_timing(device, stream)
    results["m_sweep"] = m_sweep(device, stream)

    # ---- CPU baseline on a bounded sample -------------------------------------------------------
    cpu = None
    if not args.skip_cpu:
        cpu = cpu_baseline(stress, args.cpu_seconds)

    line = {
        "metric": "ternary GEMV HBM GB/s (% peak) at M=1; prefill GEMM int8 TOPS; decode tok/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "replays": HEADLINE_REPLAYS,
        "ms_per_step": round(step_seconds * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random-init ternary weights)",
        "config": {
            "workload": "ternary GEMV M=1 cold cache: K=8192->N=28672 and K=28672->N=8192, 8 rotating copies",
            "entry_point": "gemv_plain_store (quantize + GEMV)",
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "achieved_graph": round(achieved_graph, 2),
            "frac_graph": round(achieved_graph / HBM_PEAK_GBS, 4),
            "traffic": None if not traffic or "error" in traffic else round(traffic["bytes_per_launch"]),
            "traffic_detail": traffic,
            "algorithmic_bytes_per_launch": kernel_bytes // len(kernel),
            "kernel": ("gemv_rows_kernel<0, STEPS, true, true, 1>: the launch gemv_plain_store makes, quantizing the "
                       "fp32 row in every block; two steps per row at K=8192 and seven at K=28672"),
            "prequant": {
                "kernel": "gemv_rows_kernel<0, STEPS, true, false, 1>: the same GEMV on pre-quantized activations",
                "achieved": round(prequant_achieved, 2),
                "frac": round(prequant_achieved / HBM_PEAK_GBS, 4),
                "achieved_graph": round(prequant_graph, 2),
                "frac_graph": round(prequant_graph / HBM_PEAK_GBS, 4),
                "traffic": (None if not traffic or "error" in traffic
                            else round(traffic["prequant_bytes_per_launch"])),
                "per_shape": {k: {"us": round(v["us"], 3), "GBps": round(v["GBps"], 1)}
                              for k, v in prequant_kernel.items()},
            },
            "read_ceiling": ceiling,
            "graph_frac_of_read_ceiling": round(achieved_graph / ceiling["GBps"], 4),
            "frac_of_read_ceiling_trace": (round(achieved / trace["stream_read"]["copy_launch_GBps"], 4)
                                           if trace and "copy_launch_GBps" in trace.get("stream_read", {}) else None),
            "copy_bandwidth": copy,
            "frac_of_copy_bandwidth": round(achieved / copy["GBps"], 4),
            "timing": timing,
            "per_shape": {k: {"us": round(v["us"], 3), "GBps": round(v["GBps"], 1)} for k, v in kernel.items()},
            "kernel_trace": trace,
        },
        "cpu_baseline": cpu,
        "extra": results,
    }
    print(json.dumps(line))


def decode_stack(device, generated: int = 256, repeats: int = 3, sampling=None):
    """Decode on the 24-layer d=1024 stack (vocab 32000, 36-token prompt): prefill in 32-token tiles,
    then `generated` tokens in 16-step HIP-graph bursts with one token read-back per burst.  Greedy, or
    with `sampling` = (temperature, top_k, repetition penalty) drawn by the device sampler.  tok/s counts
    the decode steps only; the wall clock includes the read-backs."""
    import hashlib

    import torch

    from ivonar_amd.decoder import StackDecoder
    from ivonar_amd.synthetic import StackConfig, decoder_stack, prompt_ids

    config = StackConfig()
    decoder = StackDecoder(decoder_stack(config, seed=1), device, burst=16, sampling=sampling is not None)
    prompt = prompt_ids(config.vocab, 36, seed=1)
    if sampling is not None:
        decoder.configure_sampling(*sampling)
    decoder.prefill(prompt)
    eager_prefill = []  # the tile program launched call by call, before capture() records it as a graph
    for _ in range(repeats):
        torch.cuda.synchronize()
        start = time.perf_counter()
        decoder.prefill(prompt)
        torch.cuda.synchronize()
        eager_prefill.append(time.perf_counter() - start)
    decoder.capture()
    tokens = decoder.generate(prompt, generated)  # warm-up, and the tokens reported
    prefill_times, decode_times = [], []
    for _ in range(repeats):
        if sampling is not None:
            decoder.configure_sampling(*sampling)
        torch.cuda.synchronize()
        start = time.perf_counter()
        decoder.prefill(prompt)
        torch.cuda.synchronize()
        middle = time.perf_counter()
        again = decoder.advance_many(generated)
        torch.cuda.synchronize()
        end = time.perf_counter()
        prefill_times.append(middle - start)
        decode_times.append(end - middle)
        if sampling is None and again[:-1] != tokens[1:]:
            raise RuntimeError("greedy decoding is not deterministic across runs")
    best = min(decode_times)
    if sampling is not None:
        return {"tok_per_s": round(generated / best, 1), "ms_per_token": round(best / generated * 1e3, 4),
                "rule": {"temperature": sampling[0], "top_k": sampling[1], "repetition_penalty": sampling[2]},
                "tokens_first8": tokens[:8]}
    return {
        "tok_per_s": round(generated / best, 1),
        "ms_per_token": round(best / generated * 1e3, 4),
        "prefill_36_ms": round(min(prefill_times) * 1e3, 3),
        "prefill_36_ms_eager": round(min(eager_prefill) * 1e3, 3),
        "prefill_note": "two 32-token tiles and the head; prefill_36_ms replays the captured tile graph once per "
                        "tile, prefill_36_ms_eager launches the same program call by call",
        "weight_bytes_per_token": decoder_bytes(config),
        "tokens_first8": tokens[:8],
        "tokens_sha1": hashlib.sha1(",".join(map(str, tokens)).encode()).hexdigest()[:16],
        "workload": f"{config.layers} layers d={config.hidden} ffn {config.dense} vocab {config.vocab}, "
                    f"36-token prompt, {generated} greedy tokens, HIP graph bursts of 16",
    }


def sampler_timing(device, stream, vocab: int = 32000) -> dict:
    """One draw of the device sampler (uniform_(), logit_bounds, sample_token) over 32000 logits,
    64 draws per HIP graph, for a few top-k values."""
    import torch

    from ivonar_amd.sampling import DeviceSampler

    sampler = DeviceSampler(vocab, device, max_top_k=1024)
    logits = torch.randn(vocab, device=device) * 3
    table = {}
    for top_k in (1, 40, 256, 1024):
        sampler.configure_sampling(temperature=0.8, top_k=top_k, repetition_penalty=1.1)

        def draw():
            sampler.uniform.uniform_()
            sampler.launch(logits)

        table[str(top_k)] = round(time_calls(draw, stream, 64, 10) * 1e6, 3)
    return {"us_per_draw_by_top_k": table, "vocab": vocab,
            "note": "uniform_ + logit_bounds + sample_token, seen cleared per top_k only"}


def decoder_bytes(config) -> int:
    """Packed weights and fp16 scales streamed per decode step (all layers and the head)."""
    h, d = config.hidden, config.dense
    per_layer = sum(rows * ((k + 3) // 4) + 2 * rows * ((k + 127) // 128)
                    for rows, k in ((3 * h, h), (h, h), (2 * d, h), (h, d)))
    return config.layers * per_layer + config.vocab * ((h + 3) // 4) + 2 * config.vocab * ((h + 127) // 128)


def cpu_model() -> str:
    """The host CPU's model name with its family/model numbers and vector extensions (a virtualised host
    may report only the brand)."""
    fields: dict[str, str] = {}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if ":" not in line:
                if fields:
                    break  # the first processor's block is enough
                continue
            key, value = (part.strip() for part in line.split(":", 1))
            fields.setdefault(key, value)
    except OSError:
        return "unknown"
    name = fields.get("model name", "unknown")
    flags = set(fields.get("flags", "").split())
    vector = [f for f in ("avx2", "avx512f", "avx512_vnni", "avx512_bf16") if f in flags]
    return f"{name} (family {fields.get('cpu family', '?')}, model {fields.get('model', '?')}; {' '.join(vector) or 'no avx2'})"


def physical_cores(allowed: set[int]) -> int:
    """Distinct (package, core) pairs among the CPUs this process may run on."""
    cores = set()
    try:
        text = Path("/proc/cpuinfo").read_text()
    except OSError:
        return len(allowed)
    for block in text.split("\n\n"):
        fields = dict(line.split(":", 1) for line in block.splitlines() if ":" in line)
        fields = {k.strip(): v.strip() for k, v in fields.items()}
        if "processor" in fields and int(fields["processor"]) in allowed:
            cores.add((fields.get("physical id", "0"), fields.get("core id", fields["processor"])))
    return len(cores) or len(allowed)


def cpu_baseline(stress, budget_seconds: float):
    """The numba GEMV restated in C++/OpenMP, timed on this host on the stress shapes: with one thread per
    physical core of this process's CPU set (at most 16), then with one thread for a quarter of the budget."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import ternary_oracle as T

    cb = T.CpuBaseline(native=True)
    allowed = os.sched_getaffinity(0) if hasattr(os, "sched_getaffinity") else set(range(os.cpu_count() or 1))
    threads = max(1, min(physical_cores(allowed), 16))
    prepared = []
    for layer, x in stress:
        planes = cb.planes_of(layer.packed, layer.in_features)
        scales = layer.scales.astype(np.float32)
        prepared.append((planes, scales, np.ascontiguousarray(x[0]), np.zeros(layer.rows, np.float32),
                         cb.workspace(layer.in_features), layer))

    def timed(count: int, budget: float) -> tuple[float, int]:
        cb.set_threads(count)
        total_bytes, total_seconds, calls = 0, 0.0, 0
        deadline = time.perf_counter() + budget
        while time.perf_counter() < deadline:
            for planes, scales, x, out, ws, layer in prepared:
                start = time.perf_counter()
                cb.gemv(x, planes, scales, None, out, ws=ws)
                total_seconds += time.perf_counter() - start
                total_bytes += gemv_bytes(1, layer.rows, layer.in_features)
                calls += 1
        return total_bytes / total_seconds / 1e9, calls

    value, calls = timed(threads, budget_seconds)
    single, single_calls = timed(1, budget_seconds / 4)
    return {
        "value": round(value, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{calls} GEMV calls over both stress shapes (~{budget_seconds:.0f} s), planes layout, OpenMP "
                  f"with {threads} threads",
        "value_1_thread": round(single, 3),
        "sample_1_thread": f"{single_calls} calls (~{budget_seconds / 4:.0f} s)",
        "cpu_model": cpu_model(),
        "cpus_allowed": len(allowed),
        "march": cb.march,
    }


if __name__ == "__main__":
    main()
