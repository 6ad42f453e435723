"""MantisNet leaf-evaluation benchmark on one MI355X.

Workload: the production MantisNet configuration
(cell_latents + cell_nodes, 5,195,909 parameters, seeded perturbed init)
evaluating B = 512 seeded random legal positions of 40-120 stones.  One step
is one full forward — trunk, value head, both cell heads and the acting-Q
composition, with the per-forward index tables derived inside the step —
over the device-resident batch.  The reference's own method is followed
(python/mantisnet/mantisnet/lab/bench.py:124-142): warm-up forwards, then
device-synchronised timed forwards; positions/s = B / (seconds per step).

The JSON line also carries
* ``roofline`` — the dominant kernel of the timed steps (largest summed
  duration among the traced kernels), its algorithmic bytes per launch over
  its average HIP-event duration on the launching stream, against 8 TB/s;
* ``seam`` — the KLENT evaluator seam (trunk + the two cell heads) on the
  same batch;
* ``cpu_baseline`` — the CPU fp32 oracle (oracle/model_ref.py, the
  restatement of the reference's CPU formulations) timed on a bounded sample
  of the same batch on this host's CPU share, plus configs[0] (B=8, smallest
  widths) with the reference's literal window-latent loops;
* ``attention`` / ``message_passing`` — the isolated-kernel configurations
  (configs[1] ragged attention, configs[2] hex message passing) with MFMA and
  HBM fractions.

Only one GPU is supported: ``--gpus N`` with N > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "hexo-shrimp-bot_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
# GPU-side spin before an isolated timing loop: the host enqueues every
# launch while the device is held, so the per-launch events bracket kernels
# that run back to back instead of host launch gaps.
HOLD_CYCLES = 20_000_000


def _hold(torch):
    torch.cuda.synchronize()
    torch.cuda._sleep(HOLD_CYCLES)


def _args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=512)
    ap.add_argument("--config", type=int, default=4, choices=(4, 5))
    ap.add_argument("--cpu-sample", type=int, default=32, help="positions in the CPU-baseline sample")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-isolated", action="store_true", help="skip the isolated attention/message-passing lines")
    ap.add_argument("--no-seam", action="store_true", help="skip the evaluator-seam timing")
    ap.add_argument("--isolated-only", action="store_true",
                    help="run only the isolated attention and message-passing lines (for kernel profiling)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only copy MIB mebibytes device-to-device once and exit (HBM counter calibration)")
    ap.add_argument("--split-cell-stages", action="store_true",
                    help="run the cell pass as two launches (the decoder sub-stage over the covered cells, then the "
                         "radius sub-stage with each chunk's stones staged on chip) instead of the fused launch")
    ap.add_argument("--no-late-game", action="store_true",
                    help="skip the configs[4] sub-line (B=1024 positions of 150-250 stones)")
    ap.add_argument("--late-steps", type=int, default=5, help="timed steps of the configs[4] sub-line")
    return ap.parse_args()


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _counters():
    """The committed rocprofv3 PMC breakdown of the forward's large kernels
    (texture address/data units, L1 stalls, L2->L1 requests, VALU and MFMA
    busy), per bench.py trace name."""
    f = ROOT / "profiles" / "counters.json"
    if f.exists():
        try:
            return json.loads(f.read_text())
        except ValueError:
            return None
    return None


def _traffic():
    """Measured HBM bytes per launch of the dominant kernel, from the
    committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, calibrated)."""
    f = ROOT / "profiles" / "traffic.json"
    if f.exists():
        try:
            return json.loads(f.read_text())
        except ValueError:
            return None
    return None


COLD_FLUSH_MIB = 512  # more than the 256 MB MALL and the L2s together


def _cold(torch, ops, dev, name, launch, reps):
    """The traced op `name` timed with the caches cold: a 512 MiB fill (not
    traced) before every launch evicts its inputs from L2 and the MALL."""
    flush = torch.empty(COLD_FLUSH_MIB * 2**20 // 4, dtype=torch.float32, device=dev)
    launch()
    with ops.trace(name) as tr:
        for _ in range(reps):
            flush.fill_(1.0)
            launch()
        torch.cuda.synchronize()
    del flush
    return tr.summary()[name]


def configs1_inputs(torch, dev):
    """The configs[1] instance: seeded lengths L ~ U{64..512} of B=256
    sequences (int32), and for fp16 then bf16 the N(0,1) q, k, v in the
    model's layout ((B, T, 8, 32) storage viewed as (B, 8, T, 32))."""
    import numpy as np

    rng = np.random.default_rng([2, 0])
    b, h, t = 256, 8, 512
    lens = torch.from_numpy(rng.integers(64, 513, b).astype(np.int32))
    gen = torch.Generator(device="cpu").manual_seed(2)
    qkv = {}
    for dtype in (torch.float16, torch.bfloat16):
        qkv[dtype] = [torch.randn(b, t, h, 32, generator=gen).to(dtype).to(dev).transpose(1, 2) for _ in range(3)]
    return lens, qkv


def configs2_inputs(torch, dev):
    """The configs[2] instance: 256 graphs, graph j the first N_j ~
    U{64..512} legal cells (engine order) of a seeded 40-120-stone position;
    (cells_qr int32 (N, 2), graph_ptr int64 (257,), x bf16 (N, 128), w bf16
    (128, 128), bias fp32 (128,)), all on dev."""
    import numpy as np

    from mantisnet import builder, synthetic

    games = synthetic.random_games(3, 256)
    cells, sizes = [], []
    for j, g in enumerate(games):
        legal, _, _ = builder.legal_moves(g)
        n = int(np.random.default_rng([3, j, 1]).integers(64, 513))
        cells.append(legal[:n])
        sizes.append(min(n, len(legal)))
    qr = torch.from_numpy(np.concatenate(cells).astype(np.int32)).to(dev)
    gptr = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)).to(dev)
    n = qr.shape[0]
    gen = torch.Generator(device="cpu").manual_seed(3)
    x = torch.randn(n, 128, generator=gen).to(torch.bfloat16).to(dev)
    # the layer's weight in the kernel's operand format once, as a model keeps
    # its parameters: no conversion between the timed launches
    w = (torch.randn(128, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16).to(dev)
    bias = (0.02 * torch.randn(128, generator=gen)).to(dev)
    return qr, gptr, x, w, bias


def isolated_attention(torch, ops, dev, reps=20):
    """B=256 sequences, L ~ U{64..512}, 8 heads, hd 32, N(0,1)."""
    lens, qkv_all = configs1_inputs(torch, dev)
    h, t = 8, 512
    res = {}
    for dtype, name in ((torch.float16, "fp16"), (torch.bfloat16, "bf16")):
        qkv = qkv_all[dtype]
        sl = lens.to(dev)
        ops.register_seq_lens(sl)
        # the longest-first work order depends on the lengths only: built once,
        # as the model builds it once per batch, and timed as its own kernel
        for _ in range(2):
            sched = ops.stone_attention_schedule(sl, h, t)
        _hold(torch)
        with ops.trace("stone_attention_schedule") as trs:
            for _ in range(5):
                sched = ops.stone_attention_schedule(sl, h, t)
        for _ in range(3):
            ops.stone_attention(*qkv, sl, schedule=sched)
        _hold(torch)
        with ops.trace("stone_attention") as tr:
            for _ in range(reps):
                ops.stone_attention(*qkv, sl, schedule=sched)
        s = tr.summary()["stone_attention"]
        c = _cold(torch, ops, dev, "stone_attention", lambda: ops.stone_attention(*qkv, sl, schedule=sched), reps)
        res[name] = {
            "avg_us": round(s["avg_us"], 2),
            "schedule_us": round(trs.summary()["stone_attention_schedule"]["avg_us"], 2),
            "tflops": round(s["tflops"], 1),
            "mfma_frac": round(s["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
            "gbps": round(s["gbps"], 1),
            "gflop_per_launch": round(s["flops_per_launch"] / 1e9, 2),
            "mb_per_launch": round(s["bytes_per_launch"] / 1e6, 1),
            "cold_avg_us": round(c["avg_us"], 2),
            "cold_mfma_frac": round(c["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
        }
    return {"config": "B=256, L~U{64..512}, H=8, hd=32, key-padding mask, no bias; warm (inputs in L2/MALL) "
                      f"and cold ({COLD_FLUSH_MIB} MiB written before each launch)", **res}


def isolated_message_passing(torch, ops, dev, reps=20):
    """256 graphs = first N_j ~ U{64..512} legal cells of seeded
    40-120-stone positions; 6-neighbour sum and mean, Linear(128,128), bf16."""
    qr, gptr, x, w, bias = configs2_inputs(torch, dev)
    n = qr.shape[0]
    nbr = ops.hex_neighbours(qr, gptr)
    for _ in range(3):
        ops.hex_aggregate_linear(x, nbr, w, bias)
    _hold(torch)
    with ops.trace("hex_aggregate_linear") as tr:
        for _ in range(reps):
            ops.hex_aggregate_linear(x, nbr, w, bias)
    s = tr.summary()["hex_aggregate_linear"]
    c = _cold(torch, ops, dev, "hex_aggregate_linear", lambda: ops.hex_aggregate_linear(x, nbr, w, bias), reps)
    ops.raise_on_device_error(dev)
    # the practical ceiling at this size: a device copy moving the same bytes
    # (half read, half written), warm, timed the same way
    half = int(s["bytes_per_launch"] // 4)
    src = torch.empty(half, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    copy_us = e0.elapsed_time(e1) * 1000.0 / reps
    del src, dst
    return {
        "config": f"256 graphs, N={n} cells, 6 axial neighbours, sum+mean then Linear(128,128), bf16; warm "
                  f"(inputs in L2/MALL) and cold ({COLD_FLUSH_MIB} MiB written before each launch)",
        "avg_us": round(s["avg_us"], 2),
        "gbps": round(s["gbps"], 1),
        "hbm_frac": round(s["gbps"] / HBM_PEAK_GBPS, 4),
        "mb_per_launch": round(s["bytes_per_launch"] / 1e6, 2),
        "cold_avg_us": round(c["avg_us"], 2),
        "cold_hbm_frac": round(c["gbps"] / HBM_PEAK_GBPS, 4),
        "copy_same_bytes_us": round(copy_us, 2),
        "copy_same_bytes_hbm_frac": round(s["bytes_per_launch"] / (copy_us * 1e3) / HBM_PEAK_GBPS, 4),
    }


def seam_timing(torch, net, bd, steps: int) -> dict:
    """The KLENT evaluator seam (klent/train.py:100-120) on the same
    device-resident batch: the policy/critic evaluation alone (trunk and the
    two cell heads, no value readout) and the whole evaluator closure,
    including both Q compositions and the copy of its three outputs to host
    memory.  Each is the median of ``steps`` device-synchronised calls."""
    from mantisnet import forward as fwd
    from mantisnet.klent.train import KlentConfig, network_evaluate

    ev = network_evaluate(net, KlentConfig(device="cuda"))

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(steps):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return round(1e3 * statistics.median(ts), 4)

    return {"policy_q_ms": timed(lambda: fwd.policy_q(net, bd)), "evaluator_ms_with_host_copy": timed(lambda: ev(bd)),
            "steps": steps}


def _host_cpus() -> dict:
    """What the host offers: logical CPUs, this process's affinity, the
    cgroup CPU quota and the CPU model."""
    info = {"host_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        info["cgroup_cpus"] = None if quota == "max" else math.ceil(int(quota) / int(period))
    except (OSError, ValueError):
        info["cgroup_cpus"] = None
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    info["cpu_model"] = model
    return info


def _cpu_threads(info: dict) -> int:
    """The CPU share this process may use: the affinity set, bounded by the
    cgroup quota and by OMP_NUM_THREADS when those are set."""
    n = info["affinity_cpus"]
    if info["cgroup_cpus"]:
        n = min(n, info["cgroup_cpus"])
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def _time_forward(fn, warmup: int, reps: int) -> float:
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline(torch, net, games, sample: int, reps: int):
    """The CPU fp32 restatement of the reference's CPU path, timed on this
    host's cores with the reference's method (lab/bench.py:124-142: warm-up
    forwards, then the median of timed forwards):

    * ``value``: the production configuration on the first ``sample``
      positions of the benchmark batch, the window-latent cycle
      vectorised (the reference's literal loops would iterate over ~676k
      windows per block at B=512);
    * ``configs0``: BASELINE configs[0] — the smallest model widths with the
      production knobs, B=8 positions of 10-40 stones — with the window-latent
      cycle as the reference's literal CPU loops, the formulation that
      reproduces the reference's own output bit for bit.
    """
    from mantisnet import MantisConfig, MantisNet, collate_positions, synthetic
    from oracle.compare import oracle_forward

    info = _host_cpus()
    threads = _cpu_threads(info)
    torch.set_num_threads(threads)
    sub = collate_positions(games[:sample])
    med = _time_forward(lambda: oracle_forward(net, sub, 0.2), 1, reps)
    tiny = MantisNet(MantisConfig(h=16, blocks=1, heads=2, value_queries=2, value_bins=5, policy_hidden=16,
                                  value_hidden=16, cell_latents=True, cell_nodes=True, cell_node_scope="all"))
    tiny.load_state_dict(synthetic.perturbed_state_dict(tiny, seed=0))
    b8 = collate_positions(synthetic.random_games(1, 8))
    med0 = _time_forward(lambda: oracle_forward(tiny, b8, 0.2, latent_loops=True), 3, 10)
    return {
        "value": round(sample / med, 2),
        "unit": "positions/s",
        "cores": threads,
        "kind": "port",
        "sample": f"configs[3]: {sample} of the {len(games)} benchmark positions, production configuration, fp32, "
                  f"window-latent cycle vectorised, median of {reps} forwards after 1 warm-up",
        "torch_threads": torch.get_num_threads(),
        **info,
        "configs0": {
            "value": round(8 / med0, 2),
            "unit": "positions/s",
            "ms_per_forward": round(1e3 * med0, 2),
            "sample": "configs[0]: B=8 positions of 10-40 stones, h=16 / 1 block / 2 heads with the production "
                      "knobs, fp32, window-latent cycle as the reference's literal loops, median of 10 after 3 "
                      "warm-ups",
        },
    }


TRACED = ("attention_substage", "cell_attention", "cell_heads", "fused_linear", "stone_attention", "run_reduce",
          "runs_to_ptr", "latent_", "row_encode", "layer_norm", "value_read", "compose_q", "gather_rows", "plan_check",
          "stable_key_order", "radius_class", "attention_slots", "covered_rows", "window_view", "segment_order",
          "radius_")


def time_workload(torch, ops, net, dev, config: int, batch_size: int, steps: int, warmup: int) -> dict:
    """One workload: seeded positions of BASELINE config ``config`` (4:
    40-120 stones, 5: 150-250), encoded and copied to the device, then
    ``warmup`` forwards, ``steps`` device-synchronised timed forwards
    (untraced: the tracer's per-launch HIP events cost host time between
    launches) and a traced pass of the same length for the per-kernel figures."""
    from mantisnet import collate_positions, synthetic

    t0 = time.perf_counter()
    games = synthetic.random_games(config, batch_size)
    t_gen = time.perf_counter() - t0
    t0 = time.perf_counter()
    batch = collate_positions(games)
    t_enc = time.perf_counter() - t0
    t0 = time.perf_counter()
    bd = batch.to(dev)
    torch.cuda.synchronize()
    t_h2d = time.perf_counter() - t0
    _log(f"config {config}: B={batch_size} cells={batch.n_cells} windows={batch.window_feat.numel()} "
         f"stones={batch.stone_own.numel()} (generate {t_gen:.2f}s, encode {t_enc:.2f}s, h2d {t_h2d:.3f}s)")
    with torch.no_grad():
        for _ in range(warmup):
            net(bd, 0.2)
        torch.cuda.synchronize()
        ops.raise_on_device_error(dev)
        _log(f"warm-up done ({warmup} steps)")
        per_step = []
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        for _ in range(steps):
            s0 = time.perf_counter()
            # a forward returns once the device has finished it: it reads the
            # device error flag (one device-to-host copy) before returning, so
            # a device-wide synchronisation per step would only add host time
            net(bd, 0.2)
            per_step.append(time.perf_counter() - s0)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t_start
        ops.raise_on_device_error(dev)
        with ops.trace(*TRACED) as tr:
            for _ in range(steps):
                net(bd, 0.2)
            torch.cuda.synchronize()
        kernels = tr.summary()
        ops.raise_on_device_error(dev)
    ms = 1e3 * elapsed / steps
    value = batch_size * steps / elapsed
    _log(f"config {config}: timed {steps} steps: {ms:.3f} ms/step, {value:.1f} positions/s")
    return {"games": games, "batch": batch, "bd": bd, "kernels": kernels, "ms": ms, "value": value,
            "per_step": per_step, "encode_s": t_enc, "h2d_s": t_h2d}


def main() -> int:
    args = _args()
    if args.gpus != 1:
        print(
            f"bench.py measures one MI355X only; --gpus {args.gpus} is not supported "
            "(the MantisNet leaf evaluation shards by position with no exchange: split the leaf batch "
            "into per-GPU sub-batches, one process per GPU, outputs concatenated in position order)",
            file=sys.stderr,
        )
        return 2
    import torch

    dev = torch.device("cuda:0")
    if args.copy_probe:
        n = args.copy_probe * 2**20 // 4
        x = torch.ones(n, dtype=torch.float32, device=dev)
        y = torch.empty_like(x)
        torch.cuda.synchronize()
        y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": 4 * n, "copy_probe_bytes_written": 4 * n}), flush=True)
        return 0

    from mantisnet import PRODUCTION, MantisNet, collate_positions, ops, synthetic

    if args.isolated_only:
        print(json.dumps({"attention": isolated_attention(torch, ops, dev),
                          "message_passing": isolated_message_passing(torch, ops, dev)}), flush=True)
        return 0

    if args.split_cell_stages:
        from mantisnet import forward as fwd

        fwd.SPLIT_CELL_STAGES = True

    torch.manual_seed(0)
    net = MantisNet(PRODUCTION)
    net.load_state_dict(synthetic.perturbed_state_dict(net, seed=0))
    net = net.to(dev).eval()

    run = time_workload(torch, ops, net, dev, args.config, args.batch, args.steps, args.warmup)
    games, batch, bd, kernels = run["games"], run["batch"], run["bd"], run["kernels"]
    ms, value, per_step = run["ms"], run["value"], run["per_step"]
    t_enc, t_h2d = run["encode_s"], run["h2d_s"]

    dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]["total_ms"])
    traffic = _traffic()
    counters = _counters()
    # the committed counters belong to one workload; other configurations report none
    if (traffic or {}).get("_workload") != {"config": args.config, "batch": args.batch}:
        traffic = None
    if (counters or {}).get("_workload") != {"config": args.config, "batch": args.batch}:
        counters = None
    roofline = {
        "kernel": dom_name,
        "bound": "hbm",
        "achieved": round(dom["gbps"], 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(dom["gbps"] / HBM_PEAK_GBPS, 4),
        "traffic": ((traffic or {}).get(dom_name) or {}).get("bytes"),
        "avg_us": round(dom["avg_us"], 2),
        "launches_per_step": dom["launches"] // args.steps,
        "share_of_step": round(dom["total_ms"] / args.steps / ms, 4),
        "traced_pass": f"{args.steps} further steps with HIP events around each traced launch",
    }
    if counters and dom_name in counters:
        # what actually binds the dominant kernel: its committed PMC breakdown
        # (the algorithmic-bytes fraction above is against HBM; the kernel is
        # bound by its gathers' path through the texture units and L1)
        roofline["limiter"] = counters[dom_name]
    line = {
        "metric": "positions evaluated/sec (MantisNet fwd, B=512)",
        "value": round(value, 2),
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "median_ms_per_step": round(1e3 * statistics.median(per_step), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded random legal positions, seeded perturbed random-init weights",
        "config": {
            "workload": f"MantisNet production forward (cell_nodes), configs[{args.config - 1}]",
            "batch_positions": args.batch,
            "stones": "40-120" if args.config == 4 else "150-250",
            "cells": int(batch.n_cells),
            "windows": int(batch.window_feat.numel()),
            "encode_s": round(t_enc, 3),
            "h2d_s": round(t_h2d, 4),
            "cell_pass": "split (decoder launch + radius launch, stones on chip)" if args.split_cell_stages
            else "fused (both cell sub-stages in one launch)",
        },
        "roofline": roofline,
        "kernels": {k: {kk: round(vv, 3) for kk, vv in v.items()} for k, v in kernels.items()},
    }
    if not args.no_late_game and args.config == 4:
        # the late-game stress batch, timed the same way (its own
        # warm-up, plain timed steps, a traced pass for the per-kernel figures)
        late = time_workload(torch, ops, net, dev, 5, 1024, args.late_steps, 2)
        kl = late["kernels"]
        ld_name, ld = max(kl.items(), key=lambda kv: kv[1]["total_ms"])
        line["configs4"] = {
            "metric": "positions evaluated/sec (MantisNet fwd, B=1024, 150-250 stones)",
            "value": round(late["value"], 2),
            "unit": "positions/s",
            "steps": args.late_steps,
            "warmup": 2,
            "ms_per_step": round(late["ms"], 4),
            "median_ms_per_step": round(1e3 * statistics.median(late["per_step"]), 4),
            "cells": int(late["batch"].n_cells),
            "windows": int(late["batch"].window_feat.numel()),
            "stones": int(late["batch"].stone_own.numel()),
            "dominant_kernel": {"kernel": ld_name, "avg_us": round(ld["avg_us"], 2),
                                "launches_per_step": ld["launches"] // args.late_steps,
                                "share_of_step": round(ld["total_ms"] / args.late_steps / late["ms"], 4),
                                "achieved_gbps": round(ld["gbps"], 1),
                                "frac_of_hbm": round(ld["gbps"] / HBM_PEAK_GBPS, 4)},
        }
        _log(f"configs[4]: {line['configs4']}")
        del late
    if not args.no_seam:
        line["seam"] = seam_timing(torch, net, bd, min(args.steps, 10))
        _log(f"seam: {line['seam']}")
    if not args.no_isolated:
        _log("isolated attention (configs[1])")
        line["attention"] = isolated_attention(torch, ops, dev)
        _log("isolated message passing (configs[2])")
        line["message_passing"] = isolated_message_passing(torch, ops, dev)
    if not args.no_cpu_baseline:
        _log(f"cpu baseline: oracle on {args.cpu_sample} positions x {args.cpu_reps}, configs[0] B=8")
        line["cpu_baseline"] = cpu_baseline(torch, net, games, args.cpu_sample, args.cpu_reps)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
