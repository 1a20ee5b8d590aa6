"""Regenerates the rocprofv3 summaries under profiles/ that bench.py's figures
come from.  Run on the GPU box from the repository root, after the library is
built:

    python3 profile_bench.py [--passes trace,traffic,counters,backward] [--out DIR]
                             [--profiles-dir DIR]

Each pass runs `rocprofv3 ... -- python3 bench.py ...` as a
child process under `timeout -s KILL`; the first pass that fails ends the
script, so no further GPU work follows a failure.  Raw rocprofv3 output goes
to --out (a scratch folder, never committed); the summaries go to profiles/
(or --profiles-dir):

  trace     kernel trace + stats of bench.py's headline (c3) and decode (c4)
            legs                        -> mha_c3_decode_c4_kernel_stats.md
  traffic   FETCH_SIZE, then WRITE_SIZE, over the same legs, calibrated on the
            bench's own 64 MiB device copies -> mha_c3_decode_c4_hbm_traffic.md,
            including the record bench.py reads for roofline.traffic (bytes per
            launch plus a digest of the kernel sources they were measured on)
  counters  two SQ counter passes over the c5 model and c2 layer legs
                                        -> flash_c5_c2_counters.md
            and over the headline step -> mha_c3_counters.md
  trainc5   SQ counters and HBM bytes of the c5 training step's attention
            kernels                     -> flash_bwd_c5_counters.md
  backward  kernel trace + stats of the c3 MHA layer backward leg
                                        -> mha_backward_c3_kernel_stats.md
  train     kernel traces of the three training-step legs
                                        -> train_step_{c1,c3_shape,c5}_kernel_stats.md
  c1        kernel trace + stats of the config-1 text model leg (forward and
            greedy generation)          -> c1_text_model_generate_kernel_stats.md
"""
from __future__ import annotations

import argparse
import collections
import csv
import datetime
import json
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import bench  # noqa: E402  (TRAFFIC_SOURCES, source_digest)

PROFILES = os.path.join(ROOT, "profiles")
PASSES = ("trace", "traffic", "counters", "trainc5", "backward", "train", "c1")
COUNTERS_A = ("GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES SQ_INSTS_VALU_MFMA_F32 "
              "SQ_INSTS_VALU SQ_INSTS_VALU_TRANS_F32 SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT")
COUNTERS_B = ("GRBM_GUI_ACTIVE SQ_WAVES SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_VALU "
              "SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS")
N_XCC, N_SIMD = 8, 1024   # MI355X: 8 XCDs, 256 CUs x 4 SIMDs


def log(msg):
    print(f"[profile_bench] {msg}", flush=True)


def short_name(name):
    n = re.sub(r"cdml::\(anonymous namespace\)::", "", name)
    n = re.sub(r"\(.*", "", n)
    return n.replace("void ", "").strip()


def run_step(cmd, timeout, log_path):
    """One GPU step under `timeout -s KILL`; returns its stdout.  rocprofv3 can
    end with a segmentation fault after the program finished and wrote its
    results: that exit is accepted when the program's JSON line was printed."""
    full = ["timeout", "-s", "KILL", str(timeout)] + cmd
    log("run: " + " ".join(cmd))
    env = dict(os.environ, TMPDIR="/tmp")
    with open(log_path, "w") as lf:
        p = subprocess.run(full, cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=lf, text=True)
    out = p.stdout
    printed = any(line.startswith("{") for line in out.splitlines())
    if p.returncode != 0 and not (p.returncode == 139 and printed):
        sys.stderr.write(out[-2000:])
        raise SystemExit(f"[profile_bench] step failed with status {p.returncode}: {' '.join(cmd)} "
                         f"(log {os.path.relpath(log_path, ROOT)})")
    return out


def rocprof(args, outdir, bench_args, timeout, log_path):
    cmd = ["rocprofv3"] + args + ["-d", outdir, "-o", "run", "--output-format", "csv", "--",
                                  "python3", "bench.py"] + bench_args
    return run_step(cmd, timeout, log_path), " ".join(["rocprofv3"] + args + [
        "-d", os.path.relpath(outdir, ROOT), "-o", "run", "--output-format", "csv", "--", "python3",
        "bench.py"] + bench_args)


def bench_line(stdout):
    for line in reversed(stdout.splitlines()):
        if line.startswith("{"):
            return json.loads(line)
    return {}


def read_stats(outdir):
    with open(os.path.join(outdir, "run_kernel_stats.csv")) as f:
        return list(csv.DictReader(f))


def read_counters(outdir):
    """{(kernel, grid): {counter: [value per dispatch]}} plus dispatch durations."""
    with open(os.path.join(outdir, "run_counter_collection.csv")) as f:
        rows = list(csv.DictReader(f))
    per = collections.defaultdict(lambda: collections.defaultdict(dict))
    for r in rows:
        key = (short_name(r["Kernel_Name"]), int(r["Grid_Size"]))
        per[key][r["Dispatch_Id"]][r["Counter_Name"]] = float(r["Counter_Value"])
        per[key][r["Dispatch_Id"]]["_ns"] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
    out = {}
    for key, disp in per.items():
        cs = collections.defaultdict(list)
        for d in disp.values():
            for c, v in d.items():
                cs[c].append(v)
        out[key] = cs
    return out


def mean(xs):
    return sum(xs) / len(xs) if xs else float("nan")


def stats_table(rows):
    lines = ["| kernel | calls | avg us | min us | max us | % time |", "|---|---|---|---|---|---|"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        lines.append(f"| `{short_name(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
    return "\n".join(lines)


def header(title, commands, note):
    return (f"# {title}\n\nWritten by `python3 profile_bench.py` on "
            f"{datetime.datetime.now(datetime.timezone.utc).strftime('%Y-%m-%d %H:%M UTC')}; "
            "the commands it ran (repository root, `TMPDIR=/tmp`):\n\n```\n" + "\n".join(commands) +
            "\n```\n\n" + note + "\n")


def write(name, text):
    with open(os.path.join(PROFILES, name), "w") as f:
        f.write(text)
    log(f"wrote profiles/{name}")


def pass_trace(out):
    d = os.path.join(out, "trace")
    so, cmd = rocprof(["--kernel-trace", "--stats"], d, ["--no-cpu-baseline", "--no-extras"], 600,
                      os.path.join(out, "trace.log"))
    b = bench_line(so)
    k = b.get("kernels_ms", {})
    note = ("The headline leg of `bench.py` (10 warm-up + 20 timed c3 MHA forward steps, then a second pass "
            "with HIP events around each kernel on the library stream) and the c4 decode leg.  The bench "
            f"line of the same run gives `value` {b.get('value')} TFLOP/s, events: flash "
            f"{k.get('flash_sdpa')} ms (`roofline.achieved` {b.get('roofline', {}).get('achieved')} TFLOP/s), "
            f"QKV with RoPE {k.get('project_qkv_rope')} ms, out-proj {k.get('out_proj')} ms; decode "
            f"{b.get('decode', {}).get('ms')} ms.  The trace averages over every launch, warm-up included.")
    write("mha_c3_decode_c4_kernel_stats.md",
          header("Kernel durations: mha_c3_decode_c4", [cmd], note) + "\n" + stats_table(read_stats(d)) + "\n")


def pass_traffic(out):
    args = ["--steps", "3", "--warmup", "1", "--no-cpu-baseline", "--no-extras"]
    cmds, got = [], {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = os.path.join(out, "traffic_" + counter.lower())
        _, cmd = rocprof(["--pmc", counter], d, args, 300, os.path.join(out, f"traffic_{counter}.log"))
        cmds.append(cmd)
        got[counter] = read_counters(d)
    # calibration: the bench's own 64 MiB (65536 KiB) device-to-device copies, grid 131072
    copy = ("__amd_rocclr_copyBuffer", 131072)
    f_cal = 65536.0 / mean(got["FETCH_SIZE"][copy]["FETCH_SIZE"])
    w_cal = 65536.0 / mean(got["WRITE_SIZE"][copy]["WRITE_SIZE"])
    rows = ["| kernel | grid | counter | dispatches | mean KiB | min KiB | max KiB |", "|---|---|---|---|---|---|---|"]
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        for (name, grid), cs in sorted(got[counter].items()):
            v = cs[counter]
            rows.append(f"| `{name}` | {grid} | {counter} | {len(v)} | {mean(v):.1f} | {min(v):.1f} | {max(v):.1f} |")

    def kib(counter, prefix):
        return sum(mean(cs[counter]) for (name, _), cs in got[counter].items() if name.startswith(prefix))

    def traffic(prefixes):
        rd = sum(kib("FETCH_SIZE", p) for p in prefixes) * f_cal
        wr = sum(kib("WRITE_SIZE", p) for p in prefixes) * w_cal
        return rd * 1024, wr * 1024

    c3, c4 = bench.C3, bench.C4
    alg_c3 = 4 * c3["batch"] * c3["seq"] * c3["dim"] * 4            # Q, K, V read, O written once
    alg_c4 = bench.decode_bytes(c4["batch"], c4["t"], c4["dim"])
    f_rd, f_wr = traffic(["flash_fwd_kernel<64"])
    d_rd, d_wr = traffic(["decode_split_kernel", "decode_combine"])
    rec = {"bytes": {"flash_c3": int(f_rd + f_wr), "decode_c4": int(d_rd + d_wr)},
           "sources": {n: bench.source_digest(p) for n, p in bench.TRAFFIC_SOURCES.items()},
           "source_files": bench.TRAFFIC_SOURCES,
           "calibration": {"fetch_size_factor": round(f_cal, 5), "write_size_factor": round(w_cal, 5)},
           "date": datetime.datetime.now(datetime.timezone.utc).strftime("%Y-%m-%d")}
    body = "\n".join(rows) + f"""

Calibration: the grid-131072 `__amd_rocclr_copyBuffer` dispatches are the bench's own
64 MiB (65536 KiB) device-to-device copies.  HBM bytes = `FETCH_SIZE` x {f_cal:.5f} +
`WRITE_SIZE` x {w_cal:.5f} (KiB per dispatch).

| kernel (c3 / c4) | read MiB | written MiB | traffic per launch | algorithmic bytes | traffic / algorithmic |
|---|---|---|---|---|---|
| `flash_fwd_kernel<64, 32, ...>` (c3, B 4, L 4096, 16 x 64) | {f_rd / 2**20:.1f} | {f_wr / 2**20:.1f} | {(f_rd + f_wr) / 1e6:.1f} MB | Q, K, V read + O written once: {alg_c3 / 1e6:.1f} MB | {(f_rd + f_wr) / alg_c3:.2f} |
| `decode_split_kernel` + `decode_combine_vec_kernel` (c4) | {d_rd / 2**20:.1f} | {d_wr / 2**20:.1f} | {(d_rd + d_wr) / 1e9:.3f} GB | K, V, q read + o written once: {alg_c4 / 1e9:.3f} GB | {(d_rd + d_wr) / alg_c4:.3f} |

The record below is what `bench.py` reports as `roofline.traffic`; it is used only while
the digest of the listed kernel sources matches the tree's.

<!-- traffic-record {json.dumps(rec)} -->
"""
    write("mha_c3_decode_c4_hbm_traffic.md",
          header("HBM traffic per dispatch: mha_c3_decode_c4", cmds,
                 "Two counter passes (one counter each, KiB per dispatch).") + "\n" + body)


def counter_table(out, tag, bench_args, keep, with_traffic=False):
    """Counter passes A and B (and FETCH_SIZE / WRITE_SIZE when with_traffic) over
    `bench.py bench_args`; one table row per kernel (and grid) whose name starts
    with one of `keep`.  Returns (commands, markdown rows)."""
    sets = [("a", COUNTERS_A), ("b", COUNTERS_B)]
    if with_traffic:
        sets += [("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE")]
    cmds, got = [], {}
    for sub, cs in sets:
        d = os.path.join(out, f"{tag}_{sub}")
        _, cmd = rocprof(["--pmc"] + cs.split(), d, bench_args, 600, os.path.join(out, f"{tag}_{sub}.log"))
        cmds.append(cmd)
        got[sub] = read_counters(d)
    a, b = got["a"], got["b"]
    head = ("| kernel | grid | dispatches | active cycles per XCC | MFMA busy / active | MFMA instr | "
            "other VALU per MFMA | of which transcendental | LDS instr per MFMA | LDS bank conflicts | "
            "waves | wave cycles waiting to issue | duration us |")
    sep = "|---|---|---|---|---|---|---|---|---|---|---|---|---|"
    if with_traffic:
        head += " HBM MB read | HBM MB written |"
        sep += "---|---|"
    rows = [head, sep]
    for key in sorted(a):
        name, grid = key
        if not name.startswith(tuple(keep)):
            continue
        ca, cb = a[key], b.get(key, {})
        act = mean(ca["GRBM_GUI_ACTIVE"]) / N_XCC
        busy = mean(ca["SQ_VALU_MFMA_BUSY_CYCLES"]) / N_SIMD
        mf = mean(ca["SQ_INSTS_VALU_MFMA_F32"])
        valu = mean(ca["SQ_INSTS_VALU"]) - mf
        trans = mean(ca["SQ_INSTS_VALU_TRANS_F32"])
        lds = mean(ca["SQ_INSTS_LDS"])
        wait = (mean(cb["SQ_WAIT_INST_ANY"]) / mean(cb["SQ_WAVE_CYCLES"])) if cb else float("nan")
        per = lambda x: f"{x / mf:.2f}" if mf else "-"
        row = (f"| `{name}` | {grid} | {len(ca['GRBM_GUI_ACTIVE'])} | {act / 1e6:.3f} M | "
               f"**{busy / act:.1%}** | {mf:,.0f} | {per(valu)} | {per(trans)} | {per(lds)} | "
               f"{mean(ca['SQ_LDS_BANK_CONFLICT']):,.0f} | {mean(cb.get('SQ_WAVES', [float('nan')])):,.0f} | "
               f"{wait:.1%} | {mean(ca['_ns']) / 1e3:.1f} |")
        if with_traffic:
            # the calibration of the traffic pass: FETCH_SIZE counts half of a 64 MiB copy's reads
            rd = mean(got["fetch"].get(key, {}).get("FETCH_SIZE", [float("nan")])) * 2 * 1024 / 1e6
            wr = mean(got["write"].get(key, {}).get("WRITE_SIZE", [float("nan")])) * 1024 / 1e6
            row += f" {rd:.1f} | {wr:.1f} |"
        rows.append(row)
    return cmds, rows


COUNTER_NOTE = ("`GRBM_GUI_ACTIVE` is summed over the 8 XCCs (divided by 8); `SQ_VALU_MFMA_BUSY_CYCLES` is "
                "summed over the 1024 SIMDs (divided by 1024) and reads 64 cycles per "
                "`v_mfma_f32_32x32x2_f32`; `SQ_INSTS_VALU` includes the MFMAs, which are subtracted; "
                "`SQ_WAIT_INST_ANY` / `SQ_WAVE_CYCLES` is the share of a wave's life spent with an "
                "instruction waiting to issue (other waves hold the SIMD, or a dependency).  Durations are "
                "under counter collection, which lengthens them.")


def pass_counters(out):
    cmds, rows = counter_table(out, "counters", ["--only", "c5_time_series_model,c2_mha_layer"], ["flash_"])
    note = ("Per dispatch of each flash-attention launch in the c5 model leg (6 layers, 256 windows x 512, "
            "8 heads x 32, causal) and the c2 layer leg (16 x 1024, 8 heads x 64, causal).  " + COUNTER_NOTE)
    write("flash_c5_c2_counters.md",
          header("Flash attention counters: c5 (d_h 32) and c2 (d_h 64)", cmds, note) + "\n" +
          "\n".join(rows) + "\n")
    cmds, rows = counter_table(out, "c3counters", ["--steps", "3", "--warmup", "1", "--no-cpu-baseline",
                                                   "--no-extras", "--no-decode"], ["flash_", "gemm_"])
    note = ("Per dispatch of the three kernels of the headline step (c3: 4 x 4096, D 1024, 16 heads x 64): "
            "the flash kernel, the Q/K/V GEMM with the RoPE epilogue and the output projection.  " +
            COUNTER_NOTE)
    write("mha_c3_counters.md",
          header("Counters of the c3 MHA forward kernels", cmds, note) + "\n" + "\n".join(rows) + "\n")


def pass_trainc5(out):
    cmds, rows = counter_table(out, "trainc5", ["--only", "c5_time_series_train_step"],
                               ["flash_bwd", "bwd_delta", "flash_fwd"], with_traffic=True)
    note = ("Per dispatch of the attention kernels of the c5 training step leg (256 windows x 512, "
            "6 layers, 8 heads x 32): the forward with row statistics, D = rowsum(dO o O), dK/dV with "
            "the dS blocks stored, and dQ over the stored blocks.  HBM bytes are FETCH_SIZE x 2 and "
            "WRITE_SIZE x 1 (KiB), the factors a 64 MiB device copy reads on those counters.  " +
            COUNTER_NOTE)
    write("flash_bwd_c5_counters.md",
          header("Attention backward counters: c5 training step", cmds, note) + "\n" + "\n".join(rows) + "\n")


def pass_backward(out):
    d = os.path.join(out, "backward")
    so, cmd = rocprof(["--kernel-trace", "--stats"], d, ["--only", "c3_mha_layer_backward"], 600,
                      os.path.join(out, "backward.log"))
    leg = bench_line(so).get("other_configs", {}).get("c3_mha_layer_backward", {})
    rc = leg.get("recomputing_statistics", {})
    note = ("The c3 MHA layer backward leg: 3 warm-up + 5 timed steps in the saved-statistics form "
            "(`cdml_sdpa_bwd_saved_rope`, the inverse RoPE of dQ and dK applied as they are stored), then the "
            "same with the statistics recomputed (`cdml_sdpa_bwd`, then `cdml_rope_qk_table`), "
            "after one `cdml_sdpa_fwd_lse`.  The bench line of the same run: attention core "
            f"{leg.get('attention_core_ms')} ms ({leg.get('attention_core_tflops')} TFLOP/s) saved, "
            f"{rc.get('attention_core_ms')} ms recomputing; whole layer backward {leg.get('ms')} ms "
            f"and {rc.get('ms')} ms.")
    write("mha_backward_c3_kernel_stats.md",
          header("Kernel durations: c3 MHA layer backward", [cmd], note) + "\n" + stats_table(read_stats(d)) + "\n")


TRAIN_LEGS = {
    "c1_text_model_train_step": ("train_step_c1_kernel_stats.md", "training step, config-1 text model "
                                 "(TrainBatchDiscrete, 4 sequences of 64 tokens)"),
    "c3_shape_train_step": ("train_step_c3_shape_kernel_stats.md", "training step, c3 shape "
                            "(TrainBatchDiscrete, 12 layers, 4 sequences of 4096 tokens)"),
    "c5_time_series_train_step": ("train_step_c5_kernel_stats.md", "training step, config 5 "
                                  "(TrainBatchContinuous, 256 windows x 512 steps)"),
}


def pass_train(out):
    for leg, (name, what) in TRAIN_LEGS.items():
        d = os.path.join(out, "train_" + leg)
        so, cmd = rocprof(["--kernel-trace", "--stats"], d, ["--only", leg], 900, os.path.join(out, leg + ".log"))
        b = bench_line(so).get("other_configs", {}).get(leg, {})
        rows = read_stats(d)
        # timed + warm-up steps the leg runs (bench.py extras)
        steps = {"c1_text_model_train_step": 20 + 5, "c3_shape_train_step": 3 + 1,
                 "c5_time_series_train_step": 3 + 1}[leg]
        total = sum(float(r["TotalDurationNs"]) for r in rows) / 1e6
        lines = ["| kernel | calls | calls/step | avg us | min us | max us | ms/step |",
                 "|---|---|---|---|---|---|---|"]
        for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
            c = int(r["Calls"])
            lines.append(f"| `{short_name(r['Name'])}` | {c} | {c / steps:g} | {float(r['AverageNs']) / 1e3:.1f} | "
                         f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                         f"{float(r['TotalDurationNs']) / 1e6 / steps:.2f} |")
        note = (f"The `{leg}` leg alone ({steps} steps in the trace, warm-up included).  The bench line of "
                f"the same run: {b.get('ms')} ms per step, {b.get('tflops')} TFLOP/s by its count.  Kernel "
                f"time summed over the trace: {total / steps:.2f} ms per step.")
        write(name, header(f"Kernel durations: {what}", [cmd], note) + "\n" + "\n".join(lines) + "\n")


def pass_c1(out):
    d = os.path.join(out, "c1")
    so, cmd = rocprof(["--kernel-trace", "--stats"], d, ["--only", "c1_text_model"], 300, os.path.join(out, "c1.log"))
    leg = bench_line(so).get("other_configs", {}).get("c1_text_model", {})
    note = ("`bench.py --only c1_text_model` builds the config-1 model (vocabulary 200, D 64, 4 heads, 2 layers, "
            "FF 128, MaxSeq 64) as a `DeviceLanguageModel` for 4 sequences and runs 100 forwards of 4 x 64 tokens "
            "(50 warm-up + 50 timed), then 6 `GenerateGreedy` calls (1 warm-up + 5 timed), each a 32-token prompt "
            "and 20 new tokens: the batched prompt prefill (embedding, 2 layers, LM head on each sequence's last "
            "row, argmax), then the other 19 greedy steps of all 4 sequences in one `tiny_decode_kernel` launch.  "
            f"The bench line of the same run: forward {leg.get('forward_ms')} ms, generation "
            f"{leg.get('generate_20_tokens_batch4_ms')} ms.")
    write("c1_text_model_generate_kernel_stats.md",
          header("Kernel durations: config-1 text model, forward and greedy generation", [cmd], note) + "\n" +
          stats_table(read_stats(d)) + "\n")


def main():
    global PROFILES
    ap = argparse.ArgumentParser()
    ap.add_argument("--passes", default=",".join(PASSES))
    ap.add_argument("--out", default=os.path.join(ROOT, "gpurun_out", "profile_bench"))
    ap.add_argument("--profiles-dir", default=PROFILES,
                    help="where the summaries go (default profiles/)")
    a = ap.parse_args()
    PROFILES = os.path.abspath(a.profiles_dir)
    os.makedirs(PROFILES, exist_ok=True)
    passes = [p for p in a.passes.split(",") if p]
    bad = set(passes) - set(PASSES)
    if bad:
        ap.error(f"unknown passes {sorted(bad)}")
    os.makedirs(a.out, exist_ok=True)
    for p in passes:
        log(f"pass {p}")
        globals()["pass_" + p](a.out)
        log(f"pass {p} done")


if __name__ == "__main__":
    main()
