"""Benchmark of the persistent GRU scan forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--kinds 0,1,2,3,4] [--no-cpu]
    python bench.py --copy-mib N [--steps K]   # counter calibration, see below

A step is one forward scan (the drop-in ``gru_scan_*`` call) over one batch
of synthetic input already resident in HBM. A second table, "train_step_ms",
times full training steps (input GEMM, scan, loss, backward) per hidden kind
at the shape of the reference's published train-step table; a third,
"calibration_forward_ms", times one calibration forward per configuration
(the scan with both hidden quantizers as min_max observers, gru_scan_observe).
The headline line is the dense
fp32 scan at T=64, B=32, H=512 (config 1, the configuration the metric is
quoted on); the other four configurations are measured in the same run and
reported under "kinds".

Per kind:
  ms_per_step  host wall time of K back-to-back calls / K (synchronised on
               both sides), i.e. what a caller of the Python API sees;
  kernel_ms    average device duration of one launch, from HIP events around
               each launch while the queue is kept ahead of the GPU, so host
               overhead is not counted (this feeds the roofline);
  host_us_per_call  host time of one call with the queue kept ahead of the
               GPU (wrapper, C entry point and HIP launch; best of 3 x 50);
  roofline     algorithmic bytes or FLOPs per launch / kernel_ms against the
               MI355X peak (HBM 8 TB/s; fp32 MFMA 157.3 TFLOP/s; for the int8
               QAT configuration, whose products run on the int8 MFMA, dense
               int8 5.0 POP/s);
  cpu_baseline the oracle (the reference's per-step PyTorch CPU path) timed on
               this host's cores on a bounded sample.

--copy-mib N runs K launches of a plain elementwise copy (out = x * 1, fp32)
of N MiB and exits. Under rocprofv3 --pmc it calibrates the FETCH_SIZE and
WRITE_SIZE counters: the copy reads and writes exactly N MiB per launch, so
the counters' ratio to N MiB scales the scan kernels' counter readings to HBM
bytes (the "traffic" field, read from profiles/traffic.json).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "gru-triton_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
INT8_MFMA_PEAK_TOPS = 5000.0  # dense int8 MFMA

# Algorithmic work per launch at the benchmark shapes (bytes: gi + out + hidden
# weights + h0 + bias; FLOPs: the hidden projection only).
WORK = {
    0: {"bytes": 16_855_040, "flops": 3 * 64 * 32 * 512, "bound": "hbm"},
    1: {"bytes": 19_994_624, "flops": 3_221_225_472, "bound": "mfma"},
    # int8 QAT: the products run on the int8 MFMA over the h levels and Wh's per-row
    # int8 codes (gs_dense_fwd_i8w), so Wh is 3 H^2 code bytes + 3H scales and the
    # peak is int8's
    2: {"bytes": 17_641_472, "flops": 3_221_225_472, "bound": "mfma", "int8": True},
    3: {"bytes": 17_635_328, "flops": 805_306_368, "bound": "mfma"},
    4: {"bytes": 537_391_104, "flops": 3_019_898_880, "bound": "hbm"},
    # single-factor Monarch (not a BASELINE.json configuration): 2 T B 3H blksz flops;
    # fp32 FMA, on the VALU in this build (fp32 vector peak = fp32 MFMA peak on MI355X)
    5: {"bytes": 17_242_112, "flops": 402_653_184, "bound": "mfma"},
    # circulant (not a BASELINE.json configuration): bytes as config 0 (Wh_circ is [3, H]);
    # flops of the circulant products done directly, 2 T B 3H H, which is how the dense
    # kernel it runs on computes them
    6: {"bytes": 16_855_040, "flops": 3_221_225_472, "bound": "mfma"},
}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def roofline(idx: int, kernel_ms: float) -> dict:
    w = WORK[idx]
    traffic = None
    try:
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get(str(idx))
    except (OSError, ValueError):
        traffic = None
    if w["bound"] == "hbm":
        achieved = w["bytes"] / (kernel_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": traffic}
    achieved = w["flops"] / (kernel_ms * 1e-3) / 1e12
    if w.get("int8"):
        # also against the fp32 MFMA peak, the bound of the same products in fp32
        return {"bound": "mfma", "achieved": round(achieved, 4), "peak": INT8_MFMA_PEAK_TOPS, "unit": "TOP/s",
                "frac": round(achieved / INT8_MFMA_PEAK_TOPS, 6), "traffic": traffic,
                "frac_of_fp32_mfma_peak": round(achieved / FP32_MFMA_PEAK_TFLOPS, 5)}
    return {"bound": "mfma", "achieved": round(achieved, 4), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 5), "traffic": traffic}


def time_kind(idx: int, steps: int, warmup: int, dev) -> dict:
    import torch

    from gru_qat_amd.configs import NAMES, SHAPES, make_config, run_config

    cfg = make_config(idx, device=dev)
    for _ in range(warmup):
        run_config(cfg)
    torch.cuda.synchronize(dev)

    # Whole-call time as a caller sees it.
    t0 = time.perf_counter()
    for _ in range(steps):
        run_config(cfg)
    torch.cuda.synchronize(dev)
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps

    # Device time per launch: keep the queue ahead of the GPU with a sleep
    # kernel, then bracket every launch with events on the launch stream.
    stream = torch.cuda.current_stream(dev)
    durs = []
    reps = max(steps, 30)
    done = 0
    while done < reps:
        n = min(50, reps - done)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        torch.cuda._sleep(int(2e7))
        for a, b in ev:
            a.record(stream)
            run_config(cfg)
            b.record(stream)
        torch.cuda.synchronize(dev)
        durs += [a.elapsed_time(b) for a, b in ev]
        done += n
    kernel_ms = statistics.mean(durs)

    # Host time per call: the same calls with the queue kept ahead of the GPU,
    # timed on the host only (what the wrapper, the C entry point and the HIP
    # launch cost the caller's thread).
    host = []
    for _ in range(3):
        torch.cuda._sleep(int(2e7))
        t0 = time.perf_counter()
        for _ in range(50):
            run_config(cfg)
        host.append((time.perf_counter() - t0) * 1e6 / 50)
        torch.cuda.synchronize(dev)
    T, B, H = SHAPES[idx]
    return {
        "name": NAMES[idx],
        "shape": {"T": T, "B": B, "H": H},
        "ms_per_step": round(wall_ms, 5),
        "kernel_ms": round(kernel_ms, 5),
        "kernel_ms_median": round(statistics.median(durs), 5),
        "host_us_per_call": round(min(host), 2),
        "tokens_per_s": round(T * B / (wall_ms * 1e-3), 1),
        "kernel_tokens_per_s": round(T * B / (kernel_ms * 1e-3), 1),
        "roofline": roofline(idx, kernel_ms),
    }


# The reference's published train-step table (README.md:163-176; fp32 at
# T=64, B=32, H=512 on an RTX 2000 Ada): variant -> ms/iter.
PUBLISHED_TRAIN_MS = {"dense": 8.8, "monarch_nb4": 5.8, "monarch_nb8": 2.0, "butterfly": 20.3, "diagonal": 1.1}


def train_steps(dev, iters: int, warmup: int) -> dict:
    """One training step per variant, as the reference's bench_triton_train.py
    (:125-137) times it: gi = F.linear(x, Wi, bi), the differentiable scan,
    loss = sum(out^2), backward into Wi, bi and the hidden parameters; the
    median over iterations of the synchronised host time. Shape (64, 32, 512),
    fp32, input size H, random weights of the reference's initial ranges."""
    import math

    import torch
    import torch.nn.functional as F

    import gru_qat_amd as G
    from gru_qat_amd.configs import Q_INT8_HIDDEN

    T, B, H = 64, 32, 512
    gen = torch.Generator().manual_seed(0)
    k = 1.0 / math.sqrt(H)

    def u(*shape, bound=k):
        return ((torch.rand(shape, generator=gen) * 2 - 1) * bound).to(dev)

    x = (torch.randn((T, B, H), generator=gen) * 0.1).to(dev)
    h0 = (torch.randn((B, H), generator=gen) * 0.1).to(dev)
    Wi, bi, bh = u(3 * H, H), u(3 * H), u(3 * H)
    variants = {
        "dense": ([u(3 * H, H)], lambda gi, p, q: G.gru_scan_persistent(gi, h0, p[0], p[-1], h_in_quant=q,
                                                                         h_out_quant=q), None),
        "dense_int8_qat": ([u(3 * H, H)], lambda gi, p, q: G.gru_scan_persistent(gi, h0, p[0], p[-1], h_in_quant=q,
                                                                                  h_out_quant=q), Q_INT8_HIDDEN),
        "monarch_nb4": ([u(3, 4, H // 4, H // 4, bound=1 / math.sqrt(H // 4))],
                        lambda gi, p, q: G.gru_scan_monarch(gi, h0, p[0], p[-1], h_in_quant=q, h_out_quant=q), None),
        "monarch_nb8": ([u(3, 8, H // 8, H // 8, bound=1 / math.sqrt(H // 8))],
                        lambda gi, p, q: G.gru_scan_monarch(gi, h0, p[0], p[-1], h_in_quant=q, h_out_quant=q), None),
        "butterfly": ([(torch.randn((3, 1, 9, H // 2, 2, 2), generator=gen) * math.sqrt(0.5)).to(dev)],
                      lambda gi, p, q: G.gru_scan_butterfly_triton(gi, h0, p[0], p[-1], h_in_quant=q, h_out_quant=q),
                      None),
        "diagonal": ([u(3, H)], lambda gi, p, q: G.gru_scan_diagonal(gi, h0, p[0], p[-1], h_in_quant=q,
                                                                       h_out_quant=q), None),
        # the whole step on this build's kernels: gs_input_proj instead of F.linear
        "dense_hip_projection": ([u(3 * H, H)], lambda gi, p, q: G.gru_scan_persistent(gi, h0, p[0], p[-1]), None),
    }
    res = {}
    for name, (hidden, scan, q) in variants.items():
        params = [torch.nn.Parameter(t.clone()) for t in [Wi, bi] + hidden + [bh]]

        project = G.input_projection if name == "dense_hip_projection" else F.linear

        def step():
            for prm in params:
                prm.grad = None
            gi = project(x, params[0], params[1])
            out = scan(gi, params[2:], q)
            out.pow(2).sum().backward()

        for _ in range(warmup):
            step()
        samples = []
        for _ in range(iters):
            torch.cuda.synchronize(dev)
            t0 = time.perf_counter()
            step()
            torch.cuda.synchronize(dev)
            samples.append((time.perf_counter() - t0) * 1e3)
        ms = statistics.median(samples)
        pub = PUBLISHED_TRAIN_MS.get(name)
        res[name] = {"ms": round(ms, 4), "reference_ms_rtx2000ada": pub,
                     "speedup_vs_reference_hw": round(pub / ms, 1) if pub else None}
    return res


def calibration_forwards(dev, kinds, iters: int, warmup: int) -> dict:
    """One calibration forward per config: gru_scan_observe with quant_h_in and
    quant_h_out as int8 symmetric min_max observers (the hidden-side work of a
    GRULayer.calibrate batch, gru_layer.py:308-336, on the per-step path
    gru_layer.py:205-223); median of HIP-event-timed calls on one stream."""
    import torch

    import gru_qat_amd as G
    from gru_qat_amd.configs import make_config

    res = {}
    for idx in kinds:
        d = make_config(idx, device=dev)
        qs = [G.FakeQuantizePerTensor(G.QuantizerConfig(mode="min_max")).to(dev) for _ in range(2)]

        def call():
            G.gru_scan_observe(d["kind"], d["gi"], d["h0"], d["w"], d["bh"], quant_h_in=qs[0], quant_h_out=qs[1],
                               hidden2=d.get("w2"))

        with torch.no_grad():
            for _ in range(warmup):
                call()
            samples = []
            for _ in range(iters):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                call()
                e1.record()
                e1.synchronize()
                samples.append(e0.elapsed_time(e1))
        res[d["name"]] = {"ms": round(statistics.median(samples), 4), "T": d["T"], "B": d["B"], "H": d["H"]}
    return res


def cpu_baseline(idx: int, budget_s: float) -> dict:
    import torch

    from gru_qat_amd.configs import make_config
    from oracle import gru_oracle as O

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    cfg = make_config(idx)
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        O.scan_config(cfg)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s or len(times) >= 50:
            break
    ms = statistics.median(times) * 1e3
    return {"value": round(ms, 3), "unit": "ms/iter", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(times)} full iterations of config {idx} (median), torch CPU restatement of the "
                      f"reference per-step path"}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kinds", default="0,1,2,3,4,5,6")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=4.0, help="seconds of CPU baseline per kind")
    ap.add_argument("--copy-mib", type=int, default=0, help="run a plain N MiB copy K times and exit")
    ap.add_argument("--no-train", action="store_true", help="skip the train-step table")
    ap.add_argument("--no-calib", action="store_true", help="skip the calibration-forward table")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(batch sharding across GPUs is not part of this build); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    import gru_qat_amd

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    if args.copy_mib > 0:
        n = args.copy_mib * (1 << 20) // 4
        x = torch.rand(n, device=dev)
        y = torch.empty_like(x)
        torch.cuda.synchronize(dev)
        for _ in range(args.steps):
            torch.mul(x, 1.0, out=y)
        torch.cuda.synchronize(dev)
        print(json.dumps({"copy_mib": args.copy_mib, "launches": args.steps,
                          "bytes_read_per_launch": 4 * n, "bytes_written_per_launch": 4 * n}), flush=True)
        return 0
    gru_qat_amd.load_library()
    kinds = [int(k) for k in args.kinds.split(",") if k.strip()]

    results = {}
    for idx in kinds:
        print(f"[bench] config {idx} ...", file=sys.stderr, flush=True)
        results[idx] = time_kind(idx, args.steps, args.warmup, dev)
        print(f"[bench] config {idx}: {json.dumps(results[idx])}", file=sys.stderr, flush=True)
    train = None
    if not args.no_train:
        print("[bench] train steps ...", file=sys.stderr, flush=True)
        train = train_steps(dev, iters=30, warmup=10)
        print(f"[bench] train steps: {json.dumps(train)}", file=sys.stderr, flush=True)
    calib = None
    if not args.no_calib:
        print("[bench] calibration forwards ...", file=sys.stderr, flush=True)
        calib = calibration_forwards(dev, kinds, iters=10, warmup=2)
        print(f"[bench] calibration forwards: {json.dumps(calib)}", file=sys.stderr, flush=True)
    faults = gru_qat_amd.workspace_faults(dev)

    cpu = {}
    if not args.no_cpu:
        for idx in kinds:
            print(f"[bench] cpu baseline config {idx} ...", file=sys.stderr, flush=True)
            cpu[idx] = cpu_baseline(idx, args.cpu_budget)
            results[idx]["cpu_baseline"] = cpu[idx]

    head = 1 if 1 in results else kinds[0]
    r = results[head]
    props = torch.cuda.get_device_properties(dev)
    line = {
        "metric": "ms/iter scan fwd at T=64,B=32,H=512 per kind; % of HBM/MFMA roofline",
        "value": r["ms_per_step"],
        "unit": "ms/iter",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded CPU generator, BASELINE.json config distributions)",
        "config": {"workload": f"config {head}: {r['name']} T={r['shape']['T']} B={r['shape']['B']} "
                               f"H={r['shape']['H']}", "kind": r["name"], **r["shape"]},
        "tokens_per_s": r["tokens_per_s"],
        "kernel_ms": r["kernel_ms"],
        "host_us_per_call": r["host_us_per_call"],
        "roofline": r["roofline"],
        "cpu_baseline": cpu.get(head),
        "kinds": {str(k): v for k, v in results.items()},
        "train_step_ms": train,
        "calibration_forward_ms": calib,
        "device": {"name": props.name, "cus": props.multi_processor_count, "host_cpu": cpu_model(),
                   "host_cores": os.cpu_count()},
        "exchange_faults": faults,
    }
    print(json.dumps(line), flush=True)
    return 0 if faults == 0 else 1


if __name__ == "__main__":
    sys.exit(main())
