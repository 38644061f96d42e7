"""Benchmark of the fused Mamba-3 inference hot path on one MI355X.

Default workload: ``fused_mamba`` at the 4 s clip shape B=16, L=400, H=16, P=64,
N=64 (R=16, Hq=1; bf16 x/B/C/z, fp32 dt/adt/trap/angles), synthetic seeded
inputs resident in HBM. A step is one call over the batch; the timed region
replays a HIP graph holding ``--steps`` back-to-back calls so host dispatch does
not stall the GPU between calls, bracketed by device synchronisation and timed
with HIP events on the launch stream, after ``--warmup`` eager calls and
untimed replays of the same graph that add up to at least 50 ms of GPU time
(so the GPU's clocks have settled whatever ``--steps`` is). The calls cycle through copies of the
inputs (each with its own output) whose total exceeds twice the 256 MB
last-level cache, so every call reads its operands from HBM; the single-set,
cache-warm time is reported beside it.

Printed as one JSON line: ``value`` is the algorithmic GB/s (unique input bytes +
output bytes per call / average call time), ``roofline`` compares it with the
8 TB/s HBM peak, ``workloads`` times the variable-length channel-folded batch
(B32 padded L400) and the 72 s long clip (B1 L7200) the same way,
``cpu_baseline`` times the CPU oracle (chunked fp32 PyTorch) on the clip
workload and on the reference's CPU-sized case and the long clip on the host
cores, ``encoder`` reports the ms per forward
of the 8-block encoder at 4 s mono x 16 with graph replay (``--no-encoder`` to
skip), and ``trifusion_model`` the same for the full TriFusion-FP model at the
reference configuration (random init; ``--no-trifusion`` to skip).
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "trifusion-fp-kernel_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
LLC_BYTES = 256 * 2**20  # MI355X last-level (Infinity) cache
WORKLOAD = dict(batch=16, time=400, heads=16, head_dim=64, state=64, rotary=16, qk_heads=1)
# other workloads are parity-test shapes; --workload times one of them instead
WORKLOADS = {
    "clip": ("fused_mamba clip B16 L400 H16 P64 N64 R16 Hq1", WORKLOAD, None),
    "long": ("fused_mamba long clip B1 L7200 H16 P64 N64 R16 Hq1 (chunk-parallel)",
             dict(WORKLOAD, batch=1, time=7200), None),
    "varlen": ("fused_mamba varlen B32 padded L400, 16 clips x 2 channel slots (lengths U{50..400}, channels "
               "U{1,2}, a mono clip's second slot length 0; seed 12) H16 P64 N64 R16 Hq1",
               dict(WORKLOAD, batch=32), (50, 12)),
}
# the reference's CPU-sized case: fp32 everything (reference tests/test_recurrence.py shapes)
CPU_WORKLOAD = dict(batch=2, time=256, heads=4, head_dim=32, state=16, rotary=4, qk_heads=1)
METRIC = "fused_mamba GB/s & %HBM peak; ms/forward 4s mono×16 encoder, 1 MI355X"
TRAFFIC_FILE = ROOT / "profiles" / "fused_mamba_clip_b16_l400_pmc.txt"
COUNTERS_FILE = ROOT / "profiles" / "fused_mamba_clip_b16_l400_counters.txt"
# sources of the clip workload's kernel; a profile summary names the hash of
# these it was measured on, and its figures are reported only if it matches
KERNEL_SOURCES = [
    ROOT / "trifusion-fp-kernel_amd" / "csrc" / name
    for name in ("mamba_pipe.hip", "mfma_tile.h", "mamba_internal.h", "common.h")
]


def parse_args():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline time budget")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-encoder", action="store_true")
    p.add_argument("--no-kernels", action="store_true", help="skip the bandwidth-kernel lines")
    p.add_argument("--kernels-only", action="store_true",
                   help="only time the bandwidth kernels at the encoder shapes (profiling aid)")
    p.add_argument("--encoder-only", action="store_true", help="only time the encoder forward (profiling aid)")
    p.add_argument("--trifusion-only", action="store_true",
                   help="only time the full TriFusion-FP model forward at 4 s mono x 16 (profiling aid)")
    p.add_argument("--no-trifusion", action="store_true", help="skip the full TriFusion-FP model timing")
    p.add_argument("--variant", default="auto", choices=["auto", "pipe", "mfma", "generic"])
    p.add_argument("--workload", default="clip", choices=sorted(WORKLOADS),
                   help="shape to time (clip: the headline B16 L400 workload)")
    p.add_argument("--eager", action="store_true", help="time Python-dispatched calls instead of graph replay")
    p.add_argument("--sets", type=int, default=0,
                   help="input sets the timed calls cycle through (0: enough to exceed twice the 256 MB "
                   "last-level cache, so operands come from HBM; 1: one set, cache-warm)")
    p.add_argument("--no-warm", action="store_true",
                   help="skip the single-set cache-warm timing (profiling aid: only cache-cold calls)")
    p.add_argument(
        "--calibrate-copy",
        type=int,
        default=0,
        metavar="MIB",
        help="only run 20 device-to-device copies of MIB MiB (HBM counter calibration) and exit",
    )
    return p.parse_args()


def calibrate_copy(torch, mib):
    """Plain copy of known size: reads and writes exactly mib MiB per copy."""
    n = mib * (1 << 20) // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes": n * 4, "copies": 20}), flush=True)


def kernel_source_hash():
    """First 16 hex digits of the SHA-256 of the clip kernel's source files."""
    import hashlib

    h = hashlib.sha256()
    for path in KERNEL_SOURCES:
        h.update(path.name.encode())
        h.update(path.read_bytes())
    return h.hexdigest()[:16]


def profile_matches(path):
    """The summary at ``path`` was measured on the current kernel source: its
    ``kernel_source_sha16:`` line equals kernel_source_hash()."""
    if not path.exists():
        return False
    for line in path.read_text().splitlines():
        if line.startswith("kernel_source_sha16:"):
            return line.split(":", 1)[1].strip() == kernel_source_hash()
    return False


def traffic_bytes():
    """HBM bytes per call from the committed rocprofv3 --pmc summary, if it was
    measured on the current kernel source."""
    if not profile_matches(TRAFFIC_FILE):
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_call:"):
            return int(line.split(":", 1)[1].strip())
    return None


def utilisation_counters():
    """MfmaUtil / VALUBusy (percent) of the clip kernel from the committed
    rocprofv3 --pmc summary, if it was measured on the current kernel source."""
    if not profile_matches(COUNTERS_FILE):
        return None
    out = {}
    for line in COUNTERS_FILE.read_text().splitlines():
        parts = line.split()
        if len(parts) >= 3 and parts[0] in ("MfmaUtil", "VALUBusy") and parts[-1] == "%":
            out[parts[0]] = float(parts[-2])
    if not out:
        return None
    out["unit"] = "percent"
    out["source"] = "profiles/" + COUNTERS_FILE.name
    return out


# Untimed GPU work before a graph's timed replay: the captured graph is
# replayed until at least this many milliseconds of it have run, whatever
# --steps is. After ~5 ms the GPU's clocks are still rising (the timed replay
# read ~2 us per call slower than after ~25 ms of replays).
WARM_GPU_MS = 50.0


def warm_graph(torch, graph, stream, min_ms=WARM_GPU_MS):
    """Replay ``graph`` (untimed) until ``min_ms`` of its GPU time has run."""
    spent = 0.0
    replays = 0
    while spent < min_ms or replays < 2:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        graph.replay()
        b.record(stream)
        b.synchronize()
        spent += a.elapsed_time(b)
        replays += 1
    return replays


def time_fused_mamba(args, torch, fused_mamba, sets, steps, warmup, variant, eager, lengths=None):
    """Average ms per call; call i reads input set i % len(sets) and writes its
    own output, so with enough sets no call finds its operands in the caches."""
    stream = torch.cuda.current_stream()
    with torch.inference_mode():
        outs = [torch.empty_like(d[2]) for d in sets]

        def call(i):
            fused_mamba(*sets[i % len(sets)], out=outs[i % len(sets)], variant=variant, lengths=lengths)

        for i in range(warmup):
            call(i)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        if eager:
            torch.cuda.synchronize()
            start.record(stream)
            for i in range(steps):
                call(i)
            end.record(stream)
            torch.cuda.synchronize()
            return start.elapsed_time(end) / steps
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for i in range(steps):
                    call(i)
        stream.wait_stream(side)
        warm_graph(torch, graph, stream)
        torch.cuda.synchronize()
        start.record(stream)
        graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_time_oracle(torch, w, budget_s, dtype):
    """Median seconds per call of the CPU oracle (chunked PyTorch) at workload
    ``w`` over a time budget (at least 3 calls), and the algorithmic bytes."""
    from oracle.recurrence import fused_mamba_chunked
    from trifusion_amd.synthetic import algorithmic_bytes, clip_inputs

    args = clip_inputs(w["batch"], w["time"], heads=w["heads"], head_dim=w["head_dim"], state=w["state"],
                       rotary=w["rotary"], qk_heads=w["qk_heads"], dtype=dtype, seed=1)
    fused_mamba_chunked(*args)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        fused_mamba_chunked(*args)
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times), algorithmic_bytes(args)


def cpu_baseline(torch, budget_s):
    """The CPU oracle on the host cores at the clip workload (the reported
    line), and at the reference's CPU-sized case and the long clip (reference
    benchmarks/benchmark_inference.py:52-65 times its cases the same way)."""
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    model = cpu_model()
    med, n, nbytes = cpu_time_oracle(torch, WORKLOAD, budget_s, torch.bfloat16)
    line = {
        "value": round(nbytes / med / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"full clip workload B16 L400 H16 P64 N64, CPU oracle (chunked fp32 PyTorch), "
        f"median of {n} calls ({med * 1e3:.1f} ms/call), {model}",
        "configs": {},
    }
    for key, w, dtype, budget in (("cpu_b2_l256_h4_p32_n16_fp32", CPU_WORKLOAD, torch.float32, budget_s / 4),
                                  ("long_b1_l7200_h16_p64_n64", dict(WORKLOAD, batch=1, time=7200), torch.bfloat16,
                                   budget_s / 2)):
        med, n, nbytes = cpu_time_oracle(torch, w, budget, dtype)
        line["configs"][key] = {"ms_per_call": round(med * 1e3, 3), "GB/s": round(nbytes / med / 1e9, 4),
                                "calls": n, "cores": threads, **w}
    return line


def graph_us(torch, fn, steps=100):
    """Average µs of ``fn(i)`` for i = 0 .. steps-1 over a replayed graph of
    ``steps`` calls (HIP events on the launch stream)."""
    stream = torch.cuda.current_stream()
    with torch.inference_mode():
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for i in range(steps):
                    fn(i)
        stream.wait_stream(side)
        warm_graph(torch, graph, stream)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e3 / steps


COLD_BYTES = 640 << 20  # input copies cycled per cold timing: 2.5x the 256 MB last-level cache


def bandwidth_kernels(torch):
    """Each single-pass kernel of the encoder at its 4 s mono x 16 shape (16 x 400
    frames, dim 512, in-proj width 2240 in rows of 2304, FFN 2 x 1365 run at
    2 x 1408): algorithmic bytes (each input element read once, each output
    written once) / time vs 8 TB/s. ``us`` repeats one input (cache-warm, as in
    a forward where the producer just wrote it); ``us_cold`` cycles through
    enough copies of the inputs that each call reads them from HBM. The first
    line, a one-element fill, is what any launch costs in this protocol."""
    from trifusion_amd.kernels import rms, swiglu
    from trifusion_amd.kernels.buffers import mamba_controls, mask_buffer
    from trifusion_amd.kernels.native import add, add_rms, mask_rms, rms_pair
    from trifusion_amd.stem import frame_audio
    from trifusion_amd.masking import masked_mean, time_mask

    g = torch.Generator(device="cuda").manual_seed(5)
    b, t, dim, proj, ffn, heads, n = 16, 400, 512, 2304, 1408, 16, 64
    rows = b * t
    w = torch.ones(dim, device="cuda")
    wn = torch.ones(n, device="cuda")
    bias = torch.zeros(heads, device="cuda")
    lengths = torch.full((b,), t, dtype=torch.int64, device="cuda")
    mask = time_mask(lengths, t)
    chans = torch.ones(b, dtype=torch.int64, device="cuda")
    bc0, ad0 = 2 * 1024, 2 * 1024 + 2 * n  # B|C columns, then the D and A columns of the in-proj output

    def x32():
        return (torch.randn(b, t, dim, device="cuda", generator=g),)

    def xb():
        return torch.randn(b, t, dim, device="cuda", generator=g), torch.randn(b, t, dim, device="cuda",
                                                                             generator=g).bfloat16()

    def pb():
        return (torch.randn(b, t, proj, device="cuda", generator=g).bfloat16(),)

    cases = [
        ("launch floor: 1-element fill", lambda: (torch.empty(1, device="cuda"),), lambda o: o.fill_(1.0), 4),
        ("rms fp32->bf16 [6400,512]", x32, lambda x: rms(x, w, out_dtype=torch.bfloat16), rows * dim * (4 + 2)),
        ("add_rms fp32+bf16 -> fp32,bf16 [6400,512]", xb, lambda x, br: add_rms(x, br, w, mask),
         rows * dim * (4 + 2 + 4 + 2) + rows),
        ("rms pair bf16 strided B|C columns [6400,2x64]", pb, lambda p: rms_pair(p[..., bc0: bc0 + 2 * n], wn, wn),
         rows * 2 * n * (2 + 2)),
        ("swiglu bf16 [6400,2816] -> [6400,1408]",
         lambda: (torch.randn(b, t, 2 * ffn, device="cuda", generator=g).bfloat16(),), lambda gu: swiglu(gu),
         rows * 3 * ffn * 2),
        ("mamba_controls bf16 [16,400,16] x2 -> fp32 [16,16,400] x2", pb,
         lambda p: mamba_controls(p[..., ad0 + heads: ad0 + 2 * heads], p[..., ad0: ad0 + heads], bias, 1e-4),
         rows * heads * (2 + 2 + 4 + 4)),
        ("masked_mean fp32 [16,400,512] -> [16,512]", x32, lambda x: masked_mean(x, lengths),
         rows * dim * 4 + b * dim * 4),
        ("mask_rows fp32 [6400,512]", x32, lambda x: mask_buffer(x, mask), rows * dim * 8 + rows),
        ("add fp32+bf16 -> fp32 [6400,512]", xb, lambda x, br: add(x, br, mask), rows * dim * (4 + 2 + 4) + rows),
        ("mask_rms bf16 -> fp32,bf16 [6400,512]", lambda: (x32()[0].bfloat16(),), lambda x: mask_rms(x, mask, w),
         rows * dim * (2 + 4 + 2) + rows),
        ("frame_audio fp32 [16,1,64000] -> bf16 [16,400,448]",
         lambda: (torch.rand(b, 1, 64000, device="cuda", generator=g) * 2 - 1,),
         lambda audio: frame_audio(audio, chans, 400, 160, 120, 448), b * 64000 * 4 + rows * 448 * 2),
    ]
    out = []
    for name, make, fn, nbytes in cases:
        one = make()
        us = graph_us(torch, lambda i: fn(*one))
        line = {"kernel": name, "us": round(us, 2), "bytes": nbytes,
                "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1), "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if nbytes > 4:
            copies = [one] + [make() for _ in range(min(255, -(-COLD_BYTES // nbytes) - 1))]
            cold = graph_us(torch, lambda i: fn(*copies[i % len(copies)]), steps=max(100, len(copies)))
            line.update({"us_cold": round(cold, 2), "frac_cold": round(nbytes / (cold * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "cold_copies": len(copies)})
            del copies
        del one
        torch.cuda.empty_cache()
        out.append(line)
    return out


def encoder_ms(torch, trifusion=False):
    """ms per forward at 4 s mono x 16 through the graph engine: the benchmark
    encoder, or with ``trifusion`` the full TriFusion-FP model at the reference
    configuration (dim 1024, 16 blocks, N=128; random init)."""
    from trifusion_amd.runtime import InferenceEngine
    from trifusion_amd.model import Encoder, ModelConfig
    from trifusion_amd.runtime import prepare_static_weights
    from trifusion_amd.trifusion import TriFusion, TriFusionConfig

    torch.manual_seed(0)
    if trifusion:
        model = TriFusion(TriFusionConfig()).eval().requires_grad_(False)
        del model.memory_head
    else:
        model = Encoder(ModelConfig()).eval().requires_grad_(False)
    prepare_static_weights(model)
    model = model.cuda()
    g = torch.Generator().manual_seed(551)
    audio = (torch.randint(-32768, 32768, (16, 1, 64000), generator=g).float() / 32768).cuda()
    lengths = torch.full((16,), 64000, dtype=torch.int64, device="cuda")
    channels = torch.ones(16, dtype=torch.int64, device="cuda")
    engine = InferenceEngine(model, graphs=True, max_graphs=1)
    engine(audio, lengths, channels)
    for _ in range(3):
        engine(audio, lengths, channels)
    torch.cuda.synchronize()
    times = []
    for _ in range(11):
        t0 = time.perf_counter()
        engine(audio, lengths, channels)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    times.sort()
    line = {"ms_per_forward": round(times[len(times) // 2] * 1e3, 4), "graph_hits": engine.graph_hits,
            "protocol": "3 warm-ups, median of 11, perf_counter + synchronize, graph replay"}
    if trifusion:
        line["model"] = "TriFusion-FP, dim 1024, 16 blocks, N=128 (528M parameters, random init, bf16 GEMMs)"
        line["reference_l4_ms_per_forward"] = 79.70  # README.md:112, an NVIDIA L4, real checkpoint
    return line


def time_workload(args, torch, fused_mamba, selected_variant, w, varlen, warm=True):
    """(ms per call cache-cold, cache-warm ms or None, algorithmic bytes, kernel
    name, input sets) of ``fused_mamba`` at workload ``w``."""
    from trifusion_amd.synthetic import algorithmic_bytes, channel_fold_lengths, clip_inputs

    host = clip_inputs(w["batch"], w["time"], heads=w["heads"], head_dim=w["head_dim"], state=w["state"],
                       rotary=w["rotary"], qk_heads=w["qk_heads"], seed=1)
    dargs = tuple(x.cuda() for x in host)
    lengths = None
    if varlen is not None:
        lengths_host, _ = channel_fold_lengths(w["batch"] // 2, w["time"], varlen[0], seed=varlen[1])
        lengths = lengths_host.cuda()
    nbytes = algorithmic_bytes(host, lengths=None if lengths is None else lengths.cpu())
    kernel = selected_variant(*dargs, variant=args.variant, lengths=lengths)
    nsets = args.sets or max(1, -(-2 * LLC_BYTES // nbytes))
    sets = [dargs] + [tuple(x.clone() for x in dargs) for _ in range(nsets - 1)]
    ms = time_fused_mamba(args, torch, fused_mamba, sets, args.steps, args.warmup, args.variant, args.eager,
                          lengths)
    warm_ms = None
    if nsets > 1 and warm:
        warm_ms = time_fused_mamba(args, torch, fused_mamba, [dargs], args.steps, args.warmup, args.variant,
                                   args.eager, lengths)
    del sets
    return ms, warm_ms, nbytes, kernel, nsets


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py runs on one GPU only: --gpus {args.gpus} is not supported "
            "(the benchmark measures one GPU; the fused recurrence would shard over (batch, head) units "
            "without collectives)",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    from trifusion_amd.mamba_fused import fused_mamba, selected_variant

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    if args.calibrate_copy:
        calibrate_copy(torch, args.calibrate_copy)
        return
    if args.encoder_only:
        print(json.dumps({"encoder": encoder_ms(torch)}), flush=True)
        return
    if args.trifusion_only:
        print(json.dumps({"trifusion_model": encoder_ms(torch, trifusion=True)}), flush=True)
        return
    if args.kernels_only:
        print(json.dumps({"bandwidth_kernels": bandwidth_kernels(torch)}), flush=True)
        return
    label, w, varlen = WORKLOADS[args.workload]
    ms, warm_ms, nbytes, kernel, nsets = time_workload(args, torch, fused_mamba, selected_variant, w, varlen,
                                                       warm=not args.no_warm)
    gbs = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded clip_inputs: x,B,C,z ~ N(0,1); dt = softplus(N(0,1)-2); A = -exp(U(0, ln16)))",
        "config": {
            "workload": label,
            "kernel": kernel,
            "timing": ("eager calls" if args.eager else f"HIP graph of {args.steps} calls, HIP events on the launch stream")
            + f", cycling through {nsets} input sets ({nsets * nbytes / 2**20:.0f} MiB)",
            "cache_warm_ms_per_step": None if warm_ms is None else round(warm_ms, 6),
            "algorithmic_bytes_per_call": nbytes,
            **w,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes() if args.workload == "clip" else None,
        },
    }
    if args.workload == "clip":
        line["roofline"]["kernel_source_sha16"] = kernel_source_hash()
        line["counters"] = utilisation_counters()
        line["workloads"] = {}
        for name in ("varlen", "long"):
            wlabel, ww, wvarlen = WORKLOADS[name]
            wms, _, wbytes, wkernel, _ = time_workload(args, torch, fused_mamba, selected_variant, ww, wvarlen,
                                                        warm=False)
            wgbs = wbytes / (wms * 1e-3) / 1e9
            line["workloads"][name] = {"workload": wlabel, "kernel": wkernel, "ms_per_call": round(wms, 6),
                                       "algorithmic_bytes_per_call": wbytes, "GB/s": round(wgbs, 2),
                                       "frac": round(wgbs / HBM_PEAK_GBS, 4)}
    if not args.no_kernels and args.workload == "clip":
        line["bandwidth_kernels"] = bandwidth_kernels(torch)
    if not args.no_encoder:
        try:
            line["encoder"] = encoder_ms(torch)
        except ImportError as err:  # encoder not built yet
            line["encoder"] = {"error": str(err)}
    if not args.no_encoder and not args.no_trifusion:
        line["trifusion_model"] = encoder_ms(torch, trifusion=True)
    if not args.no_cpu_baseline and args.workload == "clip":  # the baseline times the clip workload
        line["cpu_baseline"] = cpu_baseline(torch, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
