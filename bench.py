#!/usr/bin/env python3
"""Decode benchmark of the styx MoE hot path on one MI355X.

Workload: the 48-layer Qwen3-30B-A3B-shaped
synthetic qwen3moe -- hidden 2048, 32 q / 4 kv heads, head_dim 128,
128 experts top-8, expert FFN 768, vocab 151936, RMSNorm eps 1e-6, rope base
1e6; weights N(0, 0.02), experts mixed q4_K/q5_K/q6_K
(type(l, role) = [q4_K, q5_K, q6_K][(l + role) % 3]), attention, embedding
and LM head q8_0, all resident in HBM.  A 16-token prompt with ids uniform
in [0, 151936) (seed 0xC0FFEE) is prefilled, W warmup tokens are decoded,
then exactly K greedy decode steps are timed (one step = one full forward
pass of one token, device-side argmax, no host round trip per token).

--config k runs BASELINE.json configs[k-1] instead (numbered from 1):
  1  one qwen3moe layer, q8_0 experts (H 2048, E 128, k 8, F 768): the
     per-kernel table is the measurement (gate+up, down, reduce)
  2  the default above
  3  config 2 with a Zipf(1.1) router bias, experts in pinned host memory
     and a 6 GiB HBM budget pinned by the bias's expected popularity;
     reports the hit rate and that tokens equal the all-in-HBM run
  4  235B-A22B shape (H 4096, 94 layers, 64/4 heads, F 1536, q4_K experts)
     decoded after synthetic contexts of 512, 4096 and 32768 tokens
  5  80B-A3B MoE shape (E 512, k 10, F 512, shared expert 512, gate/up
     q4_K, down q6_K), 48 layers

The JSON line carries:
  value      decode tok/s over the K timed steps
  roofline   the dominant kernel, the fused MoE block k_moe_block (router,
             top-k, expert gate/up/down dequant-matvec, combine; k_gate_up
             when the block runs as separate kernels, --no-fuse):
             algorithmic bytes per launch / average launch time, measured
             with HIP events on the engine's stream around graph replays of
             that kernel's launches for every layer (each reading its own
             slabs, as a token does), against 8 TB/s
  cpu_baseline  the C oracle (a restatement of the reference's CPU
             dequant-then-dot path, -O2 -ffp-contract=off) decoding the same
             model on the host's cores for a bounded sample
  cpu_block  (configs 1 and 2) one MoE block of layer 0 on the oracle:
             cpu_ref_1t (1 thread) and cpu_ref_mt (16 threads), us per block
             and GB/s of its algorithmic bytes, beside the GPU block
  baseline_rows  (config 1) each of the reference's published rows of config 1 --
             the whole MoE block, gate+up+SiLU, down+reduce -- with its
             algorithmic bytes, the measured kernel time, GB/s, fraction of
             8 TB/s and the 70% target time; the fused block reports the
             first row, --no-fuse the other two
  unfused_fallbacks  times a fused launch gave up waiting and the model went
             over to the separate kernels (0 in a clean run)
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tok/s (batch 1) at 30B-A3B shape; expert matvec HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_table(m, stats: dict, timing_steps: int, graphs: bool, reps: int = 20) -> dict:
    """Per-stage table.  `avg_us` is the in-graph duration: the stage's
    launches for every layer captured as one graph and replayed `reps` times
    between two HIP events (styx_moe_time_stage), divided by the launches per
    token.  `event_us` is the eager timing pass, one HIP event pair around
    each launch (it includes each launch's dispatch, about 2 us more); it is
    also `avg_us` when graphs are off (rocprofv3 runs)."""
    out = {}
    for name, (n, ms, by) in stats.items():
        if not n:
            continue
        per_tok = max(1, round(n / timing_steps))
        ev_us = ms * 1e3 / n
        row = {"launches": int(n), "event_us": round(ev_us, 3), "bytes_per_launch": round(by / n)}
        us = ev_us
        if graphs and name != "argmax":
            rep_us, _ = m.time_stage(name, reps)
            us = rep_us / per_tok
        row["avg_us"] = round(us, 3)
        row["GB/s"] = round(by / n / (us * 1e-6) / 1e9, 1) if us > 0 else None
        out[name] = row
    return out


MB_PHASES = ["entry", "x_normalised", "limbs", "logits_seen", "ranked", "gate_up_done",
             "gu_seen", "h_limbs", "down_done", "partials_seen", "end", "gu_issued", "gu_limbs",
             "gu_dots", "gu_entered", "gu_slab"]


def moe_block_phases(m) -> dict | None:
    """Timeline of the fused MoE block on the last timed token: for each
    phase, the median and the latest workgroup (us after the layer's first
    workgroup entered), averaged over the layers."""
    tr = m.moe_block_trace()
    if tr is None:
        return None
    st, tpu = tr
    out = {}
    # slots 9 and 10 of the workgroups past the reduce ones time the next
    # layer's q/k/v folded into the tail: limbs seen, rows stored
    nred = (int(m.hp.n_embd) + 255) // 256
    per = {p: ([], []) for p in MB_PHASES + ["qkv_limbs_seen", "qkv_done"]}
    for lay in st.astype(np.float64):
        t0 = lay[:, 0][lay[:, 0] > 0].min()
        cols = [(p, lay[:, i]) for i, p in enumerate(MB_PHASES)]
        cols[9] = ("partials_seen", lay[:nred, 9])
        cols[10] = ("end", lay[:nred, 10])
        cols += [("qkv_limbs_seen", lay[nred:, 9]), ("qkv_done", lay[nred:, 10])]
        for p, c in cols:
            v = c[c > 0]
            if len(v):
                per[p][0].append(np.median(v - t0) / tpu)
                per[p][1].append((v.max() - t0) / tpu)
    for p, (med, mx) in per.items():
        if med:
            out[p] = {"median_us": round(float(np.mean(med)), 2),
                      "last_us": round(float(np.mean(mx)), 2)}
    return out


AT_PHASES = ["entry", "q_rotated", "tiles_done", "partials_stored", "partials_seen", "end"]


def attn_phases(m) -> dict | None:
    """Timeline of the attention launch on the last timed token: for each
    phase, the median and the latest workgroup (us after the layer's first
    workgroup entered), averaged over the layers; and the active chunks."""
    tr = m.attn_trace()
    if tr is None:
        return None
    st, tpu = tr
    per = {p: ([], []) for p in AT_PHASES}
    chunks = []
    for lay in st.astype(np.float64):
        live = lay[lay[:, 7] > 0]
        if not len(live):
            continue
        t0 = live[:, 0].min()
        chunks.append(int(live[0, 6]))
        for i, p in enumerate(AT_PHASES):
            v = live[:, i][live[:, i] > 0]
            if len(v):
                per[p][0].append(np.median(v - t0) / tpu)
                per[p][1].append((v.max() - t0) / tpu)
    if not chunks:
        return None
    out = {"active_chunks": chunks[-1], "workgroups": int((st[-1][:, 7] > 0).sum())}
    for p, (med, mx) in per.items():
        if med:
            out[p] = {"median_us": round(float(np.mean(med)), 2),
                      "last_us": round(float(np.mean(mx)), 2)}
    return out


def cpu_baseline(m, prompt, seconds: float, threads: int) -> dict:
    """Oracle decode of the same model on host cores (bounded sample)."""
    from oracle import oracle as O
    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import oracle_from_model

    t0 = time.perf_counter()
    orc = oracle_from_model(m, n_ctx=len(prompt) + 256)
    log(f"cpu baseline: exported model to host in {time.perf_counter() - t0:.1f}s")
    O.set_threads(threads)
    n, pos, tok = 0, 0, int(prompt[0])
    gen = []  # greedy tokens: argmax after the last prompt token, then after each of them
    t0 = time.perf_counter()
    while True:
        logits, *_ = orc.forward(pos, tok)
        n += 1
        pos += 1
        if pos >= len(prompt):
            tok = O.argmax(logits)
            gen.append(tok)
        else:
            tok = int(prompt[pos])
        el = time.perf_counter() - t0
        if el >= seconds or pos >= orc.n_ctx:
            break
    return {"value": round(n / el, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} full forward passes (prompt then greedy) of the same model, "
                      f"{el:.1f}s, C oracle with {threads} OpenMP threads",
            "host": host_info(threads)}, gen


def cpu_block_baseline(m, seconds: float) -> dict:
    """One MoE block (ffn norm, router, top-k, k expert gate/up/SiLU/down,
    weighted combine) of layer 0 on the oracle, single-threaded (cpu_ref_1t)
    and with 16 threads (cpu_ref_mt): us per block over a bounded number of
    repetitions (about `seconds` each), and GB/s of its algorithmic bytes
    (router, the routed slabs, the vectors)."""
    from oracle import oracle as O
    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import oracle_from_model
    orc = oracle_from_model(m, n_ctx=8)
    hp = m.hp
    rng = np.random.default_rng(0x1234)
    x = rng.standard_normal(hp.n_embd).astype(np.float32)
    _, _, _, ids, _ = orc.moe_block(0, x)
    names = ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps")
    slab = sum(orc.t[f"blk.0.{n}.weight"][2].nbytes // hp.n_expert for n in names)
    H, F, E, k = hp.n_embd, hp.n_ff_exp, hp.n_expert, hp.n_expert_used
    nbytes = k * slab + E * H * 4 + 4 * (2 * H + 2 * k * F + 2 * H)
    out = {"bytes_per_block": int(nbytes), "experts": ids.tolist()}
    for label, thr in (("cpu_ref_1t", 1), ("cpu_ref_mt", 16)):
        O.set_threads(thr)
        orc.moe_block(0, x)
        n, t0 = 0, time.perf_counter()
        while True:
            orc.moe_block(0, x)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        us = el / n * 1e6
        out[label] = {"us_per_block": round(us, 1), "GB/s": round(nbytes / us / 1e3, 3),
                      "threads": thr, "blocks": n}
    out["host"] = host_info(16)
    out["kind"] = "port: C++ restatement of the reference's CPU dequant+matvec path"
    return out


def baseline_rows(table: dict) -> dict:
    """The reference's published config-1 rows: the kernel time measured here
    beside the algorithmic bytes, the fraction of 8 TB/s and the 70% target."""
    rows = {}

    def row(label, stages):
        got = [table[s] for s in stages if s in table]
        if len(got) != len(stages):
            return
        by = sum(g["bytes_per_launch"] for g in got)
        us = sum(g["avg_us"] for g in got)
        rows[label] = {"kernels": list(stages), "bytes": by, "avg_us": round(us, 3),
                       "GB/s": round(by / us / 1e3, 1), "frac": round(by / us / 1e3 / HBM_PEAK_GBS, 4),
                       "target_70pct_us": round(by / (0.7 * HBM_PEAK_GBS) / 1e3, 3)}
    row("moe_block", ["moe_block"])
    row("moe_block_separate", ["router", "moe_gate_up", "moe_down", "reduce"])
    row("gate_up_silu", ["moe_gate_up"])
    row("down_reduce", ["moe_down", "reduce"])
    return rows


def host_info(threads: int) -> dict:
    """The host the CPU baseline ran on: logical CPUs the process may use
    and in all, the CPU model and socket count from lscpu, the OpenMP
    threads used."""
    import subprocess
    info = {"omp_threads": threads, "nproc": len(os.sched_getaffinity(0)),
            "logical_cpus": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() == "Model name":
                info["model_name"] = v.strip()
            elif k.strip() == "Socket(s)":
                info["sockets"] = int(v.strip()) if v.strip().isdigit() else v.strip()
            elif k.strip() == "Core(s) per socket":
                info["cores_per_socket"] = int(v.strip()) if v.strip().isdigit() else v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def copy_probe(nbytes: int) -> int:
    """One plain copy of nbytes between two HBM buffers: its HBM counters
    should read nbytes fetched and nbytes written."""
    from styx_amd import Gpu
    gpu = Gpu(0)
    src, dst = gpu.zeros(nbytes), gpu.buffer(nbytes)
    gpu.sync()
    src.copy_to(dst, 0, 0, nbytes)
    gpu.sync()
    log(f"copy probe: {nbytes} bytes")
    src.free(), dst.free()
    gpu.close()
    return 0


def stream_read_gbs(gpu, nbytes: int = 2 << 30, reps: int = 10) -> tuple[float, int]:
    """Achievable HBM streaming-read bandwidth: styx_op_read_probe (each
    workgroup a contiguous chunk, 8 non-temporal dwordx4 loads in flight per
    lane) over a 2 GiB buffer, wall clock over `reps` back-to-back launches,
    at 1024 to 16384 workgroups of 256; the best rate and its grid."""
    from styx_amd import _lib as L
    grids = (1024, 2048, 4096, 8192, 16384)
    buf, out = gpu.buffer(nbytes), gpu.buffer(max(grids) * 4 * 4)
    lib = gpu.lib
    best = (0.0, 0)
    for g in grids:
        L.check(lib.styx_op_read_probe(gpu.h, buf.ptr, nbytes, out.ptr, g))
        gpu.sync()
        t0 = time.perf_counter()
        for _ in range(reps):
            L.check(lib.styx_op_read_probe(gpu.h, buf.ptr, nbytes, out.ptr, g))
        gpu.sync()
        el = time.perf_counter() - t0
        best = max(best, (nbytes * reps / el / 1e9, g))
    buf.free(), out.free()
    return best


# Kernels whose HBM traffic is measured on config 2, with their algorithmic
# bytes per launch (means over the 48 layers of configs[1]):
#   k_moe_block  router E*H*4 + 8 slots x (gate + up + down slab) + 16*H
#   k_gate_up    8 slots x (gate + up slab) + limbs, logits, outputs
TRAFFIC_KERNELS = {
    # router + 8 slots x (gate + up + down) + vectors, and the next layer's
    # q/k/v (5120 q8_0 rows of 2048: 2176 B each) in 47 of the 48 launches
    "k_moe_block": ("moe_block", 128 * 2048 * 4 + 8 * 3256320 + 16 * 2048 + 47 * 5120 * 2176 // 48),
    "k_gate_up": ("moe_gate_up", 17423616),
}


def traffic_json(stage: str) -> Path:
    return ROOT / "profiles" / f"{stage}_traffic_30b_a3b.json"


def pmc_commands(kernel: str) -> list[str]:
    b = ("python -u bench.py --steps 4 --warmup 1 --timing-steps 1 --no-cpu-baseline "
         "--no-graph")
    return [
        "rocprofv3 --pmc FETCH_SIZE --kernel-include-regex copyBuffer --output-format csv "
        "-d OUT -o copy_fetch -- python -u bench.py --copy-probe 268435456",
        "rocprofv3 --pmc WRITE_SIZE --kernel-include-regex copyBuffer --output-format csv "
        "-d OUT -o copy_write -- python -u bench.py --copy-probe 268435456",
        f"rocprofv3 --pmc FETCH_SIZE --kernel-include-regex {kernel} --output-format csv "
        f"-d OUT -o k_fetch -- {b}",
        f"rocprofv3 --pmc WRITE_SIZE --kernel-include-regex {kernel} --output-format csv "
        f"-d OUT -o k_write -- {b}",
    ]


def traffic_from_profile(stage: str) -> dict | None:
    """HBM bytes per launch of the stage's kernel on config 2, measured with
    rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE) and scaled by the copy-kernel
    calibration (``--traffic-from``)."""
    p = traffic_json(stage)
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text())
    except ValueError:
        return None


def pmc_values(path: Path, name_re: str) -> list[float]:
    import csv
    with open(path) as f:
        return [float(r["Counter_Value"]) for r in csv.DictReader(f)
                if re.search(name_re, r["Kernel_Name"])]


def traffic_from(out_dir: str, kernel: str) -> int:
    """Reduce the four pmc_commands(kernel) outputs (under out_dir) to HBM
    bytes per launch of `kernel`.  FETCH_SIZE and WRITE_SIZE read KiB per
    dispatch; each is scaled by bytes / (counter x 1024) of a plain copy of
    known size, then the per-dispatch sum is averaged over every dispatch of
    the kernel in the run (all layers, so all expert type triples of the
    configs[1] model)."""
    if kernel not in TRAFFIC_KERNELS:
        raise SystemExit(f"bench.py: no algorithmic byte count for {kernel}")
    stage, algo = TRAFFIC_KERNELS[kernel]
    d = Path(out_dir)
    n = 268435456
    cf = pmc_values(d / "copy_fetch_counter_collection.csv", "copyBuffer")
    cw = pmc_values(d / "copy_write_counter_collection.csv", "copyBuffer")
    gf = pmc_values(d / "k_fetch_counter_collection.csv", kernel)
    gw = pmc_values(d / "k_write_counter_collection.csv", kernel)
    if len(cf) != 1 or len(cw) != 1 or not gf or len(gf) != len(gw):
        raise SystemExit(f"bench.py: unexpected PMC rows in {d}")
    ff, wf = n / (cf[0] * 1024), n / (cw[0] * 1024)
    fetch, write = float(np.mean(gf)), float(np.mean(gw))
    per = fetch * 1024 * ff + write * 1024 * wf
    rec = {"kernel": f"{kernel} (all layers of the configs[1] model)",
           "bytes_per_launch": int(round(per)), "algorithmic_bytes_per_launch": algo,
           "traffic_over_algorithmic": round(per / algo, 4),
           "fetch_kib_per_dispatch_mean": round(fetch, 2),
           "write_kib_per_dispatch_mean": round(write, 2), "dispatches": len(gf),
           "calibration": {"copy_bytes": n, "copy_fetch_kib": cf[0], "copy_write_kib": cw[0],
                           "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)},
           "commands": pmc_commands(kernel)}
    traffic_json(stage).write_text(json.dumps(rec, indent=1) + "\n")
    log(json.dumps(rec))
    return 0


def config_setup(k: int, layers: int | None):
    """(synth config, workload text, extra model options) of config k."""
    from dataclasses import replace
    from styx_amd import CFG_30B_A3B, CFG_LAYER_Q8, SynthConfig
    from styx_amd import _lib as L
    if k == 1:
        cfg, text = CFG_LAYER_Q8, ("configs[0]: one qwen3moe layer (H 2048, 32/4 heads, E 128, "
                                   "top-8, F 768), q8_0 experts and attention, vocab 4096")
    elif k in (2, 3):
        cfg = CFG_30B_A3B
        text = ("configs[1]: 48-layer Qwen3-30B-A3B-shaped synthetic qwen3moe, experts mixed "
                "q4_K/q5_K/q6_K, attention/embedding/head q8_0, all resident in HBM; greedy "
                "decode after a 16-token prompt")
        if k == 3:
            cfg = replace(cfg, router_zipf_s=1.1)
            text = ("configs[2]: configs[1] with a Zipf(1.1) router bias, experts in pinned host "
                    "memory, 6 GiB HBM expert budget pinned by expected popularity, cold slabs "
                    "read in place from host memory by the fused MoE block (--arena: gathered "
                    "into the HBM arena in-stream)")
    elif k == 4:
        cfg = SynthConfig(n_layers=94, n_embd=4096, n_heads=64, n_kv_heads=4, head_dim=128,
                          n_expert=128, n_expert_used=8, n_ff_exp=1536,
                          exp_type=(L.Q4_K, L.Q4_K, L.Q4_K))
        text = ("configs[3]: 94-layer Qwen3-235B-A22B shape (H 4096, 64/4 heads, E 128, top-8, "
                "F 1536), q4_K experts, q8_0 attention/head; decode after synthetic contexts")
    elif k == 5:
        cfg = SynthConfig(n_layers=48, n_embd=2048, n_heads=16, n_kv_heads=2, head_dim=128,
                          n_expert=512, n_expert_used=10, n_ff_exp=512, n_ff_shexp=512,
                          exp_type=(L.Q4_K, L.Q4_K, L.Q6_K))
        text = ("configs[4]: 48-layer 80B-A3B MoE shape (H 2048, E 512, top-10, F 512, shared "
                "expert 512), gate/up q4_K, down q6_K")
    else:
        raise SystemExit(f"bench.py: unknown --config {k}")
    if layers:
        cfg = replace(cfg, n_layers=layers)
    return cfg, text


def expected_popularity_csv(m, path: Path) -> None:
    """Popularity input for config 3: the Zipf bias b_e = -s ln(rank) makes
    expert e about exp(b_e) times as likely; hits = round(1e6 exp(b_e))."""
    rows = ["layer,expert,hits"]
    for l in range(m.hp.n_layers):
        _, _, data = m.export_tensor(f"blk.{l}.ffn_gate_inp.bias")
        b = data.view(np.float32)
        rows += [f"{l},{e},{int(round(1e6 * np.exp(b[e])))}" for e in range(len(b))]
    path.write_text("\n".join(rows) + "\n")


def zipf_report(m, n_tok: int) -> dict:
    """Routing statistics (the HUD of generate_moe.rs:87-119) of n_tok
    tokens drawn uniformly from the vocabulary and forwarded one by one (a
    random model's greedy stream soon cycles through a few tokens, so it
    would measure its own cycle, not the router's popularity), then of as
    many greedy decode steps: the hit rate against the HBM hot set on each,
    and the popularity the router bias produced on the random tokens --
    each layer's experts ranked by their bias, picks per token of each rank
    over all layers, the least-squares exponent of picks vs rank over the
    ranks picked on fewer than half the tokens, the share of picks among
    the 41 top ranks (the hot slots a 6 GiB budget holds per layer at this
    shape)."""
    L, E, k = m.hp.n_layers, m.hp.n_expert, m.hp.n_expert_used
    rank_of = np.empty((L, E), np.int64)
    for l in range(L):
        b = m.export_tensor(f"blk.{l}.ffn_gate_inp.bias")[2].view(np.float32)
        rank_of[l, np.argsort(-b, kind="stable")] = np.arange(E)
    picks = np.zeros(E, np.int64)
    rng = np.random.default_rng(0x21FF)
    hot = cold = 0
    for t in rng.integers(0, m.hp.n_vocab, n_tok):
        m.forward_token(int(t), want_logits=False)
        ids = m.last_expert_ids().astype(np.int64)
        for l in range(L):
            picks[rank_of[l, ids[l]]] += 1
        hc = m.last_hot_cold()
        hot += int(hc[:, 0].sum())
        cold += int(hc[:, 1].sum())
    ghot = gcold = 0
    for _ in range(n_tok):
        m.decode(1)
        hc = m.last_hot_cold()
        ghot += int(hc[:, 0].sum())
        gcold += int(hc[:, 1].sum())
    per_tok = picks / (n_tok * L)
    r = np.arange(1, E + 1)
    sel = (per_tok < 0.5) & (per_tok > 0)
    slope = float(np.polyfit(np.log(r[sel]), np.log(per_tok[sel]), 1)[0]) if sel.sum() > 2 else None
    return {"hit_rate": round(ghot / max(ghot + gcold, 1), 4),
            "hit_rate_random_tokens": round(hot / max(hot + cold, 1), 4),
            "routing_tokens": n_tok,
            "zipf_fitted_exponent": None if slope is None else round(-slope, 3),
            "top41_pick_share": round(float(picks[:41].sum() / picks.sum()), 4),
            "rank1_picks_per_token": round(float(per_tok[0]), 4),
            "picks_by_rank": picks.tolist()}


def gather_report(m, table: dict, extra: dict) -> dict:
    """Cold-slab traffic of the arena placement: the cold slabs per layer at
    the measured hit rate, the gather launch's event time in the timed
    tokens (on the copy stream, overlapping the hot slots' expert kernels),
    and host-pinned -> HBM rates of the gather kernel alone over k slabs of
    each tensor and of the copy engine (SDMA, hipMemcpyAsync) moving as many
    bytes."""
    from styx_amd import _lib as L
    k, slab = m.hp.n_expert_used, m.slab_bytes
    cold = k * (1.0 - extra["hit_rate"])
    out = {"cold_slabs_per_layer": round(cold, 3)}
    g = table.get("gather")
    if g:
        out["in_token_gather_us_per_layer"] = g["event_us"]
    gpu = m.gpu
    import ctypes as C
    # the gather kernel alone (styx_op_gather_slabs) on k slabs of each of the
    # three tensors' sizes, host-pinned -> HBM, against the copy engine
    sizes = [slab // 3 // 16 * 16] * 3
    srcs = [gpu.buffer(k * sz, L.BUF_HOST_PINNED) for sz in sizes]
    dsts = [gpu.buffer(k * sz) for sz in sizes]
    ids = gpu.from_numpy(np.arange(k, dtype=np.int32))
    sp = (C.c_void_p * 3)(*[b.ptr for b in srcs])
    dp = (C.c_void_p * 3)(*[b.ptr for b in dsts])
    sl = (C.c_int64 * 3)(*sizes)

    def gather():
        L.check(gpu.lib.styx_op_gather_slabs(gpu.h, sp, sl, dp, sl, ids.ptr, k, 0))
    gather()
    gpu.sync()
    t0 = time.perf_counter()
    for _ in range(5):
        gather()
    gpu.sync()
    el = (time.perf_counter() - t0) / 5
    out["kernel_gather_h2d_GBps"] = round(k * sum(sizes) / el / 1e9, 2)
    n = k * sum(sizes)
    src, dst = gpu.buffer(n, L.BUF_HOST_PINNED), gpu.buffer(n)
    src.copy_to(dst, 0, 0, n)
    t0 = time.perf_counter()
    for _ in range(5):
        src.copy_to(dst, 0, 0, n)
    el = (time.perf_counter() - t0) / 5
    out["sdma_h2d_GBps"] = round(n / el / 1e9, 2)
    for b in srcs + dsts + [src, dst, ids]:
        b.free()
    return out


def measure(m, args, prompt):
    """Prefill, warmup, K timed greedy steps, then per-launch timing steps.
    Returns (tok/s, seconds, greedy tokens produced after the first)."""
    gpu = m.gpu
    t0 = time.perf_counter()
    for t in prompt:
        m.forward_token(int(t), want_logits=False)
    log(f"prefill {len(prompt)} tokens in {time.perf_counter() - t0:.3f}s")
    toks = [m.decode(args.warmup)] if args.warmup else []
    gpu.sync()
    t0 = time.perf_counter()
    toks.append(m.decode(args.steps))
    gpu.sync()
    el = time.perf_counter() - t0
    log(f"decode {args.steps} steps in {el:.4f}s = {args.steps / el:.1f} tok/s; "
        f"first tokens {toks[-1][:8].tolist()}")
    m.set_timing(True)
    m.kernel_stats_reset()
    toks.append(m.decode(args.timing_steps))
    stats = m.kernel_stats()
    m.set_timing(False)
    phases = moe_block_phases(m)
    aph = attn_phases(m)
    table = kernel_table(m, stats, args.timing_steps, not args.no_graph)
    if phases:
        table["moe_block"]["phases"] = phases
    if aph and "attn" in table:
        table["attn"]["phases"] = aph
    return args.steps / el, el, np.concatenate(toks), table


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", type=int, default=2, help="config number k, 1-5: BASELINE.json configs[k-1] (default 2)")
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--timing-steps", type=int, default=16,
                    help="extra decode steps run with per-launch HIP event timing")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--cpu-block-seconds", type=float, default=3.0,
                    help="configs 1-2: seconds of each single-block oracle timing (1 and 16 "
                         "threads)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--layers", type=int, default=None, help="(testing only) fewer layers")
    ap.add_argument("--contexts", default="512,4096,32768",
                    help="config 4: synthetic context lengths to decode after")
    ap.add_argument("--arena", action="store_true",
                    help="configs[2]: gather cold slabs into the HBM arena (the MoE block then "
                         "runs as separate kernels) instead of reading them in place from host "
                         "memory inside the fused block")
    ap.add_argument("--routing-tokens", type=int, default=128,
                    help="configs[2]: greedy tokens whose routing gives the hit rate and the "
                         "fitted popularity exponent")
    ap.add_argument("--no-fuse", action="store_true",
                    help="run the MoE block as four kernels instead of the fused launch")
    ap.add_argument("--no-fold-qkv", action="store_true",
                    help="launch each layer's q/k/v matvec separately instead of folding it into "
                         "the previous layer's fused MoE block")
    ap.add_argument("--no-graph", action="store_true",
                    help="enqueue kernels one by one instead of replaying a HIP graph per token")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run one device-to-device copy of BYTES (the calibration kernel "
                         "for rocprofv3 FETCH_SIZE/WRITE_SIZE) and exit")
    ap.add_argument("--traffic-from", default=None, metavar="DIR",
                    help="only reduce the rocprofv3 --pmc outputs in DIR (copy calibration and "
                         "the kernel's FETCH_SIZE/WRITE_SIZE) into the HBM-traffic record and exit")
    ap.add_argument("--traffic-kernel", default="k_moe_block", choices=sorted(TRAFFIC_KERNELS),
                    help="kernel of --traffic-from")
    args = ap.parse_args()
    if args.traffic_from:
        return traffic_from(args.traffic_from, args.traffic_kernel)
    if args.copy_probe:
        return copy_probe(args.copy_probe)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the MoE decode path is "
              "single-GPU; its sharding across GPUs is a design, not built here)", file=sys.stderr)
        return 2

    from styx_amd import Gpu, MoeModel

    cfg, workload = config_setup(args.config, args.layers)
    rng = np.random.default_rng(0xC0FFEE)
    prompt = rng.integers(0, cfg.n_vocab, 16).astype(np.uint32)
    n_ctx = len(prompt) + args.warmup + args.steps + args.timing_steps + 8
    if args.config == 3:
        n_ctx += 2 * args.routing_tokens

    gpu = Gpu(0)
    stream_gbs, stream_grid = stream_read_gbs(gpu)
    log(f"streaming-read probe: {stream_gbs:.1f} GB/s over 2 GiB ({stream_grid} workgroups)")
    extra = {}
    t0 = time.perf_counter()
    if args.config == 4:
        ctxs = [int(c) for c in args.contexts.split(",") if c]
        m = MoeModel.synth(gpu, cfg, n_ctx=max(ctxs) + n_ctx, use_graph=not args.no_graph,
                           fuse=not args.no_fuse, fold_qkv=not args.no_fold_qkv)
    else:
        m = MoeModel.synth(gpu, cfg, n_ctx=max(n_ctx, 512), use_graph=not args.no_graph,
                           fuse=not args.no_fuse, fold_qkv=not args.no_fold_qkv)
    log(f"built synthetic model in {time.perf_counter() - t0:.1f}s on {gpu.name}: "
        f"{m.hp.expert_bytes_hbm / 2**30:.2f} GiB experts in HBM, slab {m.slab_bytes} B")

    if args.config == 3:
        # the all-in-HBM run with the same bias is the reference stream
        value_hbm, _, toks_hbm, _ = measure(m, args, prompt)
        hist = Path(os.environ.get("TMPDIR", "/tmp")) / f"styx_zipf_hist_{os.getpid()}.csv"
        expected_popularity_csv(m, hist)
        m.close()
        t0 = time.perf_counter()
        m = MoeModel.synth(gpu, cfg, n_ctx=max(n_ctx, 512), use_graph=not args.no_graph,
                           fuse=not args.no_fuse, fold_qkv=not args.no_fold_qkv,
                           expert_budget_mb=6144, expert_hist=str(hist),
                           arena=args.arena)
        log(f"host-pinned model in {time.perf_counter() - t0:.1f}s: "
            f"{m.hp.expert_bytes_hbm / 2**30:.2f} GiB hot in HBM, "
            f"{m.hp.expert_bytes_host / 2**30:.2f} GiB in host memory")
        extra["all_in_hbm_tok_s"] = round(value_hbm, 3)

    if args.config == 4:
        per_ctx = {}
        for c in ctxs:
            m.reset()
            m.fill_kv(c)
            args_c = argparse.Namespace(**vars(args))
            args_c.warmup = min(args.warmup, 4)
            v, el, toks, table = measure(m, args_c, prompt[:1])
            per_ctx[str(c)] = {"tok_s": round(v, 3), "ms_per_step": round(1e3 * el / args.steps, 4),
                               "kernels": table}
            log(f"context {c}: {v:.1f} tok/s")
        value, el = per_ctx[str(ctxs[-1])]["tok_s"], None
        el = args.steps / value
        table = per_ctx[str(ctxs[-1])]["kernels"]
        extra["contexts"] = per_ctx
        toks = None
    else:
        value, el, toks, table = measure(m, args, prompt)
    for k, v in table.items():
        log(f"  {k:18s} {v}")

    if args.config == 3:
        extra["tokens_equal_all_in_hbm"] = bool(np.array_equal(toks, toks_hbm))
        extra.update(zipf_report(m, args.routing_tokens))
        hist.unlink(missing_ok=True)
        if args.arena:
            extra["gather"] = gather_report(m, table, extra)

    # the dominant kernel: the fused MoE block, or gate/up when the block
    # runs as separate kernels
    stage = "moe_block" if "moe_block" in table else "moe_gate_up"
    kname = {"moe_block": "k_moe_block (MoE block: router, expert gate/up/down dequant-matvec, "
                          "combine)",
             "moe_gate_up": "k_gate_up (expert gate+up dequant-matvec)"}[stage]
    gu = table.get(stage, {})
    roofline = None
    if gu:
        ach = gu["GB/s"]
        tr = traffic_from_profile(stage) if args.config == 2 else None
        roofline = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(ach / HBM_PEAK_GBS, 4),
                    "traffic": tr["bytes_per_launch"] if tr else None,
                    "stream_read_GBps": round(stream_gbs, 1),
                    "frac_of_stream_read": round(ach / stream_gbs, 4),
                    "kernel": kname,
                    "bytes_per_launch": gu["bytes_per_launch"], "avg_us": gu["avg_us"],
                    "launches": gu["launches"]}

    cpu = None
    if not args.no_cpu_baseline and args.config in (1, 2, 5):
        m.reset()
        threads = min(16, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
        cpu, gen = cpu_baseline(m, prompt, args.cpu_seconds, threads)
        log(f"cpu baseline: {cpu}")
        # the GPU stream starts one token after the oracle's first greedy token
        n_cmp = min(len(gen) - 1, len(toks))
        extra["greedy_tokens_verified"] = n_cmp
        extra["greedy_identical"] = bool(np.array_equal(np.asarray(gen[1:1 + n_cmp], np.uint32),
                                                        toks[:n_cmp]))
        log(f"greedy stream vs oracle: {n_cmp} tokens, identical={extra['greedy_identical']}")

    if args.config in (1, 2) and not args.no_cpu_baseline:
        extra["cpu_block"] = cpu_block_baseline(m, args.cpu_block_seconds)
        stg = table.get("moe_block") or table.get("moe_gate_up")
        if stg and args.config == 1:
            extra["cpu_block"]["gpu_us_per_block"] = sum(
                table[s]["avg_us"] for s in ("moe_block", "moe_gate_up", "moe_down", "reduce",
                                             "router") if s in table)
        log(f"cpu block: {extra['cpu_block']}")
    if args.config == 1:
        extra["baseline_rows"] = baseline_rows(table)
    extra["unfused_fallbacks"] = m.unfused_fallbacks()

    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(1e3 * el / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": workload, "n_layers": cfg.n_layers, "hidden": cfg.n_embd,
                   "experts": cfg.n_expert, "top_k": cfg.n_expert_used,
                   "expert_ffn": cfg.n_ff_exp, "vocab": cfg.n_vocab, "batch": 1,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": table,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)
    m.close()
    gpu.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
