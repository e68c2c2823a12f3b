"""Benchmark of the fused LNCC loss hot path on one MI355X.

One step = ``fused_lncc_loss(pred, target, 7).backward()`` with ``pred.grad = None`` first, on the
headline workload (2,16,128,128,128) fp32, k=7 (target ~ N(0,1) seed 0, pred = 0.8 target +
0.6 N(0,1) seed 1; CPU-generated, resident in HBM before timing). Prints one JSON line:

* value / unit: algorithmic HBM throughput of the whole step, 12 B per voxel (read pred, read
  target, write grad once) / ms_per_step, in GB/s;
* roofline: the fused kernel alone (lncc_fused_kernel; lncc_small_kernel for volumes of at most
  16^3), timed with HIP events on the stream it is launched on, against the 8 TB/s HBM peak; traffic = FETCH_SIZE + WRITE_SIZE per launch from the
  committed rocprofv3 counter summary when present;
* order: one untimed step (one-time host costs), a clock settle (the fused kernel, untimed, for
  --settle-ms of GPU time), the kernel-only timing, then --warmup untimed steps and exactly
  --steps timed steps, with no idle gap between them, so that every timed region runs at the
  clock a busy GPU keeps;
* cpu_baseline: the reference's naive PyTorch LNCC (dense grouped conv3d + autograd, restated in
  oracle/torch_lncc_port.py) on the host cores: one of the 32 volumes of the headline workload
  (the whole (1,1,32^3) k=3 case with --workload cpu), with the thread count, os.cpu_count() and
  the CPU model.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _sub in ("fused-lncc_amd", "oracle", os.path.join("tests", "golden")):
    sys.path.insert(0, os.path.join(ROOT, _sub))

HBM_PEAK_GBS = 8000.0
BYTES_PER_VOXEL = {"float32": 12, "bfloat16": 6}
METRIC = "fwd+bwd ms & achieved HBM GB/s (% of peak), (2,16,128³) fp32 k=7, 1 GPU"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "lncc_fused_kernel_headline_pmc.json")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="headline",
                    choices=["headline", "bf16", "mri", "large", "cpu", "feat16", "feat64"])
    ap.add_argument("--kernel-reps", type=int, default=40)
    ap.add_argument("--settle-ms", type=float, default=150.0,
                    help="untimed GPU work (the fused kernel) before anything is timed, so that every "
                         "timed region runs at the settled clock; 0 = none")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--target-grad", action="store_true",
                    help="time the step with the optional target-side gradient as well "
                         "(fused_lncc_loss(..., target_grad=True)); 16 B/voxel fp32, 8 B/voxel bf16")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 268 MB device-to-device copy (calibrates HBM byte counters)")
    return ap.parse_args()


def copy_probe():
    """A plain copy kernel of known size: 2^26 float32 read + 2^26 float32 written per launch."""
    import torch
    x = torch.randn(1 << 26, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(5):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": x.numel() * 4, "copy_probe_bytes_written": y.numel() * 4}))


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_baseline(workload, k, seconds):
    """The reference's naive PyTorch path (oracle/torch_lncc_port.py) on the host threads torch
    uses: the whole (1,1,32^3) k=3 case for the cpu workload, otherwise a sample of the workload's
    (N,C) volumes (one 128^3 volume of the headline, bf16 and large workloads, in fp32; the
    MRI-shaped volume whole; 32 of the 256 16^3 volumes of feat16; one 64^3 volume of feat64),
    timed until ``seconds`` of work or 50 runs, median."""
    import torch

    import torch_lncc_port
    import workloads as wl
    spec = wl.WORKLOADS[workload]
    sample = {"cpu": spec["shape"], "mri": spec["shape"], "feat16": (1, 32, 16, 16, 16), "feat64": (1, 1, 64, 64, 64)}
    shape = sample.get(workload, (1, 1, 128, 128, 128))
    p, t = wl.make_inputs(workload, shape)
    p, t = p.float(), t.float()
    for _ in range(2 if workload == "cpu" else 0):   # warm-up of the tiny case
        torch_lncc_port.loss_and_grad(p, t, k)
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        torch_lncc_port.loss_and_grad(p, t, k)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() >= t_end or len(times) >= 50:
            break
    times.sort()
    med = times[len(times) // 2]
    vox = 1
    for n in shape:
        vox *= n
    nvol = spec["shape"][0] * spec["shape"][1]
    what = "the whole workload" if workload == "cpu" else (
        "the volume" if workload == "mri" else f"{shape[0] * shape[1]} of the {nvol} volumes")
    threads = torch.get_num_threads()
    return {"value": round(vox * 12 / med / 1e9, 6), "unit": "GB/s", "cores": threads,
            "kind": "port", "ms": round(med * 1e3, 4), "voxels_per_s": round(vox / med, 1),
            "os_cpu_count": os.cpu_count(), "torch_threads": threads, "cpu_model": _cpu_model(),
            "sample": f"{what}, {tuple(shape)} fp32 k={k}, loss + grad wrt pred; median of "
                      f"{len(times)} runs = {med * 1e3:.3f} ms ({vox / med / 1e6:.3f} Mvoxel/s) on "
                      f"{threads} threads (os.cpu_count() = {os.cpu_count()}) of {_cpu_model()}"}


def main():
    a = parse()
    if a.copy_probe:
        copy_probe()
        return
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {a.gpus} requested). The loss is "
              "independent per (N,C) volume; multi-GPU use is data-parallel with no collective in "
              "the loss.", file=sys.stderr)
        sys.exit(2)
    import torch

    import workloads as wl
    from fused_lncc import _lib, fused_lncc_loss

    spec = wl.WORKLOADS[a.workload]
    k = spec["k"]
    p, t = wl.make_inputs(a.workload)
    dev = torch.device("cuda:0")
    p = p.to(dev).requires_grad_(True)
    t = t.to(dev).requires_grad_(a.target_grad)
    dtname = str(p.dtype).replace("torch.", "")
    V = p.numel()
    torch.cuda.synchronize()

    def step():
        p.grad = None
        t.grad = None
        fused_lncc_loss(p, t, k, target_grad=a.target_grad).backward()

    # the fused kernel alone, through the C ABI on the current stream
    lib = _lib.load()
    B = spec["shape"][0] * spec["shape"][1]
    D, H, W = spec["shape"][2:]
    code = _lib.FL_BF16 if p.dtype == torch.bfloat16 else _lib.FL_F32
    nbytes = lib.fl_workspace_bytes(B, D, H, W, k)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    grad = torch.empty_like(p)
    grad_t = torch.empty_like(t) if a.target_grad else None
    loss_buf = torch.empty(1, device=dev)
    stream = torch.cuda.current_stream(dev)

    def kernel():
        if a.target_grad:   # both gradients: the one fused launch (k <= 7) and the loss finalize
            _lib.check(lib.fl_lncc_loss_grad_pt(p.data_ptr(), t.data_ptr(), code, B, D, H, W, k, 1e-5,
                                                loss_buf.data_ptr(), grad.data_ptr(), grad_t.data_ptr(),
                                                ws.data_ptr(), nbytes, stream.cuda_stream))
        else:
            _lib.check(lib.fl_lncc_fused_partials(p.data_ptr(), t.data_ptr(), code, B, D, H, W, k, 1e-5,
                                                  grad.data_ptr(), ws.data_ptr(), nbytes, stream.cuda_stream))

    # Clock settle. The first step pays one-time host costs (torch loads the code of its fill
    # kernel, the autograd engine starts its device thread: ~25 ms with the GPU idle), so it runs
    # first. A GPU that has been idle starts at a low clock and needs ~30 ms of load to reach its
    # steady state (the first launches of the headline kernel take 480-560 us against 425 us), so
    # batches of the kernel then run until settle_ms of GPU time have passed (at most 4000
    # launches). None of it is timed; its length is reported.
    step()
    torch.cuda.synchronize()
    settled_ms, launches = 0.0, 0
    while settled_ms < a.settle_ms and launches < 4000:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(10):
            kernel()
        e1.record(stream)
        e1.synchronize()
        settled_ms += e0.elapsed_time(e1)
        launches += 10

    # kernel time: HIP events around each launch, on the stream it is launched on
    kev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * a.kernel_reps)]
    kwarm = 10
    for i in range(a.kernel_reps + kwarm):
        if i >= kwarm:
            kev[2 * (i - kwarm)].record(stream)
        kernel()
        if i >= kwarm:
            kev[2 * (i - kwarm) + 1].record(stream)
    torch.cuda.synchronize()
    kms = [kev[2 * i].elapsed_time(kev[2 * i + 1]) for i in range(a.kernel_reps)]
    kernel_ms = sum(kms) / len(kms)
    del grad, grad_t, ws

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(a.steps + 1)]
    evs[0].record()
    for i in range(a.steps):
        step()
        evs[i + 1].record()
    torch.cuda.synchronize()
    total_ms = evs[0].elapsed_time(evs[-1])
    per = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(a.steps))
    ms_per_step = total_ms / a.steps
    median_ms = per[len(per) // 2]

    # algorithmic bytes: with the target gradient, one more gradient is written
    step_bpv = BYTES_PER_VOXEL[dtname] + (BYTES_PER_VOXEL[dtname] // 3 if a.target_grad else 0)
    step_bytes = V * step_bpv
    alg_bytes = step_bytes
    achieved = alg_bytes / (kernel_ms * 1e-3) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE) and not a.target_grad:
        with open(TRAFFIC_FILE) as f:
            prof = json.load(f)
        if prof.get("workload") == a.workload:
            traffic = prof.get("hbm_bytes_per_launch")

    out = {
        "metric": (METRIC if a.workload == "headline" and not a.target_grad else
                   f"fwd+bwd{' (pred and target gradients)' if a.target_grad else ''} GB/s, "
                   f"{a.workload} {spec['shape']} k={k}"),
        "value": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "settle_ms": round(settled_ms, 1),
        "ms_per_step": round(ms_per_step, 5),
        "median_ms": round(median_ms, 5),
        "kernel_ms": round(kernel_ms, 5),
        "voxels_per_s": round(V / (ms_per_step * 1e-3), 1),
        "pct_of_hbm_peak": round(100.0 * step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",  # the arithmetic type of the path; bf16 inputs are widened on load (config.input_dtype)
        "data": "synthetic",
        "config": {"workload": f"lncc fwd+bwd {a.workload}", "shape": list(spec["shape"]), "kernel_size": k,
                   "input_dtype": dtname, "bytes_per_voxel": step_bpv, "target_grad": a.target_grad},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": traffic,
                     "kernel": ("lncc_small_kernel" if max(D, H, W) <= 16 else "lncc_fused_kernel") +
                               (" (both gradients, with the loss finalize)" if a.target_grad else ""),
                     "algorithmic_bytes_per_launch": alg_bytes},
    }
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(a.workload, k, a.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
