"""Per-stage timing of the pipelined recurrence kernel.

Runs ``fused_mamba`` (variant ``pipe``) at the clip workload B16 L400 H16 P64
N64 R16, or with ``--varlen`` at the channel-fold batch (B32 padded L400, 16
clips x 2 channel slots, lengths U{50..400}, a mono clip's second slot length
0, seed 12), with the library built with ``-DTF_STAGE_PROBE`` (``python -m
trifusion_amd.build --stage-probe``, on the build host) and prints what its
stage markers recorded:

* workgroup 0, per role wave (0-3 output, 4-7 state, 8-11 prologue): the
  stages of its third chunk iteration and of the walk's start, in shader
  clock cycles (``s_memtime``) from the start of that iteration;
* the length of every chunk iteration (output wave 0: interval A start to
  the end of interval B's barrier);
* every workgroup's duration (``s_memrealtime``, 100 MHz): by XCD, head and
  batch row, by chunk count with a least-squares fit duration = fixed +
  per-chunk cost, the kernel's span and the sum of workgroup times over
  256 CUs.

The markers keep their timestamps in registers and store them once after
the walk, so the kernel issues no extra memory operation while it walks.

Usage: ``python -m trifusion_amd.stage_probe [--cold] [--varlen]``; ``--cold``
runs 11 other input sets first, so that the probed call reads its operands from
HBM.
"""

import argparse
import collections
import ctypes
import statistics

import torch

from trifusion_amd import _lib, build
from trifusion_amd.synthetic import channel_fold_lengths, clip_inputs

TIME, HEADS, CUS = 400, 16, 256
ROLES = ["out0", "out1", "out2", "out3", "st0", "st1", "st2", "st3", "pro0", "pro1", "pro2", "pro3"]
ITERATION_EVENTS = {
    0: "A start", 13: "gate done", 1: "rotary done", 2: "scores done", 3: "controls done", 4: "A end",
    5: "A barrier", 8: "score.v done", 9: "gated", 6: "state done", 7: "phase done", 11: "B end", 12: "B barrier",
}
START_EVENTS = {20: "kernel start", 16: "loads issued", 17: "before controls", 14: "start barrier in",
                15: "start barrier out"}


def run(cold, varlen=False):
    if not build.STAGE_PROBE_LIB_PATH.exists():
        raise RuntimeError(f"{build.STAGE_PROBE_LIB_PATH} is missing: build it with "
                           "'python -m trifusion_amd.build --stage-probe' first")
    _lib.LIB_PATH = build.STAGE_PROBE_LIB_PATH
    from trifusion_amd import fused_mamba

    lib = _lib.load()
    lib.tf_stage_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.tf_stage_probe_read.restype = ctypes.c_int
    dev = torch.device("cuda")
    batch = 32 if varlen else 16
    lengths = channel_fold_lengths(batch // 2, TIME, 50, seed=12)[0].to(dev) if varlen else None
    args = tuple(a.to(dev) for a in clip_inputs(batch, TIME, heads=HEADS, seed=1))
    out = torch.empty_like(args[2])
    with torch.inference_mode():
        if cold:
            for k in range(11):
                other = tuple(a.to(dev) for a in clip_inputs(batch, TIME, heads=HEADS, seed=50 + k))
                fused_mamba(*other, out=torch.empty_like(other[2]), lengths=lengths, variant="pipe")
        else:
            for _ in range(3):
                fused_mamba(*args, out=out, lengths=lengths, variant="pipe")
        torch.cuda.synchronize()
        fused_mamba(*args, out=out, lengths=lengths, variant="pipe")
    torch.cuda.synchronize()
    ts = (ctypes.c_longlong * (12 * 64))()
    blk = (ctypes.c_longlong * (4096 * 3))()
    _lib.check(lib.tf_stage_probe_read(ts, blk), "tf_stage_probe_read")
    return [[ts[w * 64 + k] for k in range(64)] for w in range(12)], list(blk), batch * HEADS


def report(ts, blk, cold, units=256):
    varlen = units > 256
    name = "varlen channel-fold batch B32" if varlen else "clip workload B16"
    lines = [f"{name} L{TIME} H{HEADS} P64 N64 R16, variant pipe, "
             f"{'cache-cold (11 other input sets first)' if cold else 'cache-warm (3 calls first)'}"]
    if any(ts[w][0] for w in range(12)):
        lines += _stage_tables(ts)
    else:
        lines.append("workgroup 0 walked fewer than three chunk iterations: no stage table")
    return "\n".join(lines + _workgroups(blk, units))


def _stage_tables(ts):
    lines = []
    t0 = min(ts[w][0] for w in range(12) if ts[w][0])
    lines.append("workgroup 0, third chunk iteration: cycles from its start (-1: the role has no such stage)")
    lines.append(f"{'':>18}" + "".join(f"{r:>7}" for r in ROLES))
    for k, name in ITERATION_EVENTS.items():
        row = [ts[w][k] - t0 if ts[w][k] else -1 for w in range(12)]
        if any(v >= 0 for v in row):
            lines.append(f"{name:>18}" + "".join(f"{v:7d}" for v in row))
    lines.append("workgroup 0, the walk's start: cycles from the same origin")
    for k, name in START_EVENTS.items():
        lines.append(f"{name:>18}" + "".join(f"{ts[w][k] - t0 if ts[w][k] else -1:7d}" for w in range(12)))
    lines.append(f"walk end (last wave): {max(ts[w][21] for w in range(12)) - t0} cycles")
    lines.append("chunk iterations (output wave 0): interval A start -> interval B barrier end, cycles")
    for j in range(12):
        a, b = ts[0][24 + j], ts[0][40 + j]
        if not a:
            break
        lines.append(f"  iteration {j}: {b - a:6d}")
    return lines


def _workgroups(blk, units):
    start = [blk[3 * i] for i in range(units)]
    end = [blk[3 * i + 1] for i in range(units)]
    dur = [(e - s) * 10 for s, e in zip(start, end)]  # ns at 100 MHz
    unit = [blk[3 * i + 2] // 256 for i in range(units)]
    chunks = [blk[3 * i + 2] % 256 for i in range(units)]
    first = min(start)
    lines = [f"workgroups: {units}; start spread {(max(start) - first) * 10} ns; span (first start to last end) "
             f"{(max(end) - first) * 10} ns; duration min {min(dur)} median {statistics.median(dur):.0f} "
             f"max {max(dur)} ns; sum of durations / {CUS} CUs {sum(dur) / CUS:.0f} ns"]
    lines.append("  median by XCD (workgroup % 8): "
                 + " ".join(f"{statistics.median(dur[x::8]):.0f}" for x in range(8)))
    by_head = collections.defaultdict(list)
    by_batch = collections.defaultdict(list)
    by_chunks = collections.defaultdict(list)
    for i in range(units):
        by_head[unit[i] % HEADS].append(dur[i])
        by_batch[unit[i] // HEADS].append(dur[i])
        by_chunks[chunks[i]].append(dur[i])
    lines.append("  median by head: " + " ".join(f"{statistics.median(by_head[h]):.0f}" for h in sorted(by_head)))
    lines.append("  median by batch row: " + " ".join(f"{statistics.median(by_batch[b]):.0f}"
                                                     for b in sorted(by_batch)))
    lines.append("  by chunk count: " + "; ".join(f"{c}: {len(v)} x {statistics.median(v):.0f}"
                                                  for c, v in sorted(by_chunks.items())))
    walked = [(c, d) for c, d in zip(chunks, dur) if c > 0]
    if len({c for c, _ in walked}) > 1:
        mc = statistics.fmean(c for c, _ in walked)
        md = statistics.fmean(d for _, d in walked)
        slope = sum((c - mc) * (d - md) for c, d in walked) / sum((c - mc) ** 2 for c, _ in walked)
        lines.append(f"  fit over walked units: duration = {md - slope * mc:.0f} ns + {slope:.0f} ns per chunk")
    return lines


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--cold", action="store_true", help="read the probed call's operands from HBM")
    parser.add_argument("--varlen", action="store_true", help="the channel-fold batch instead of the clip")
    opts = parser.parse_args(argv)
    ts, blk, units = run(opts.cold, opts.varlen)
    print(report(ts, blk, opts.cold, units), flush=True)


if __name__ == "__main__":
    main()
