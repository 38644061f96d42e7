"""The stage-probe report (trifusion_amd/stage_probe.py) on synthetic
timestamps: every stage a role records appears with its offset from the third
iteration's start, stages a role does not have read -1, iteration lengths are
B-barrier end minus A start, and workgroup durations are grouped by the unit
and chunk count each workgroup recorded, with a least-squares fixed +
per-chunk cost."""

from trifusion_amd import build, stage_probe


def _synthetic():
    ts = [[0] * 64 for _ in range(12)]
    for w in range(12):
        ts[w][0] = 1000 + w  # third iteration's A start
        ts[w][5] = 4000      # A barrier
        ts[w][12] = 6000     # B barrier
        ts[w][20] = 100      # kernel start
        ts[w][21] = 9000     # walk end
        for k in (16, 14, 15):
            ts[w][k] = 200 + k
    for w in range(4, 8):
        ts[w][1] = 2500      # state waves' rotary
    ts[11][17] = 300         # prologue wave 3 before the controls
    for j in range(3):  # 0 marks an event that was not recorded
        ts[0][24 + j] = 500 + 1000 * j
        ts[0][40 + j] = 500 + 1000 * j + 700 + j
    blk = [0] * (4096 * 3)
    for i in range(256):
        unit = (i % 8) * 32 + i // 8
        chunks = 1 + unit % 7
        blk[3 * i] = 5
        # 2 us + 1 us per chunk, head 3 slower by 1 us (100 MHz ticks)
        blk[3 * i + 1] = 5 + 200 + 100 * chunks + (100 if unit % 16 == 3 else 0)
        blk[3 * i + 2] = unit * 256 + chunks
    return ts, blk


def test_report_tables():
    ts, blk = _synthetic()
    lines = stage_probe.report(ts, blk, cold=True).splitlines()
    assert "cache-cold" in lines[0]
    rotary = next(line for line in lines if line.strip().startswith("rotary done")).split()[2:]
    assert [int(v) for v in rotary] == [-1] * 4 + [2500 - 1000] * 4 + [-1] * 4
    a_bar = next(line for line in lines if line.strip().startswith("A barrier")).split()[2:]
    assert [int(v) for v in a_bar] == [3000] * 12
    before_ctl = next(line for line in lines if line.strip().startswith("before controls")).split()[2:]
    assert [int(v) for v in before_ctl] == [-1] * 11 + [300 - 1000]
    iters = [line for line in lines if line.strip().startswith("iteration ")]
    assert [int(line.split()[-1]) for line in iters] == [700, 701, 702]
    by_chunks = next(line for line in lines if "by chunk count" in line)
    assert "7: " in by_chunks and "1: " in by_chunks
    fit = next(line for line in lines if "fit over walked units" in line)
    rhs = fit.split("=")[1]  # " <fixed> ns + <per chunk> ns per chunk"
    fixed = float(rhs.split("ns")[0])
    per_chunk = float(rhs.split("+")[1].split("ns")[0])
    assert abs(per_chunk - 1000) < 30 and abs(fixed - 2000) < 150


def test_probe_library_is_separate():
    assert build.STAGE_PROBE_LIB_PATH != build.LIB_PATH
    assert build.STAGE_PROBE_LIB_PATH.name == "libtrifusion_amd_stage_probe.so"
