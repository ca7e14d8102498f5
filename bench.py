"""Benchmark of the greedy token loop (predict_token_by_token on ids) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3b32] [--no-cpu]

One step is one full mitok_generate call on the workload: the prompt forward
of every sequence plus (n_new - 1) cached decode steps, greedy ids chosen on
the device, only ids copied back.  Inputs (seeded weights, prompts) are
resident before the timed region.  The timed region is bracketed by device
synchronisation; `value` is generated tokens per second (batch x n_new per
step).  Prints ONE JSON line.

Besides the timed region the run measures, with HIP events on the library's
stream, the average duration of the dominant kernel class (roofline), and
times the CPU oracle on a bounded sample of the same workload (cpu_baseline).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import rustcrates_amd as ra  # noqa: E402
from rustcrates_amd import configs, seeded  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
FP64_MFMA_PEAK_TFS = 78.6  # MI355X dense FP64 matrix, TFLOP/s


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def workload_prompt(w):
    lens = configs.prompt_lengths(w)
    return seeded.prompts(w.prompt_seed, lens, w.model.vocab, max_len=w.prompt_len), np.array(lens, np.uint32)


def time_generate(net, prompt, lens, n_new, steps, warmup):
    for _ in range(warmup):
        net.generate(prompt, lens=lens, n_new=n_new)
    ra.device_synchronize(0)
    t0 = time.perf_counter()
    pre = dec = 0.0
    ids = None
    for _ in range(steps):
        ids = net.generate(prompt, lens=lens, n_new=n_new)
        t = net.last_timings()
        pre += t["prefill_ms"]
        dec += t["decode_ms"]
    ra.device_synchronize(0)
    wall = time.perf_counter() - t0
    return wall, pre / steps, dec / steps, ids


def kernel_class(net, prompt, lens, n_new, cls, reps=2):
    """HIP-event totals of one kernel class over `reps` generate calls (direct launches)."""
    net.timing_enable(cls)
    for _ in range(reps):
        net.generate(prompt, lens=lens, n_new=n_new)
    r = net.timing_read()
    net.timing_enable(0)
    return r


def prefill_flops(w, lens):
    """Algorithmic flops of the prompt pass: 8 per complex multiply-add of the
    Q/K/V and FFN products over every prompt row, the causal half of Re(q.k)
    (8 per key) and of P.V (4, real x complex), and the vocab product of each
    sequence's last row only."""
    c = w.model
    rows = float(sum(lens))
    proj = 8.0 * c.layers * rows * (3 * c.d * c.d + 2 * c.d * c.ffn)
    attn = c.layers * sum(12.0 * c.d * s * (s + 1) / 2 for s in lens)
    vocab = 8.0 * len(lens) * c.d * c.vocab
    return proj + attn + vocab


def decode_step_bytes(c, lens, n_new):
    """HBM bytes of one decode step averaged over the generation: every weight
    once (plus the vocab bias), and per sequence and layer the K and V rows of
    the cache, the new token's K, V and the Re(bias_pos) row 0 entries."""
    weights = 16.0 * c.weight_elems() + 16.0 * c.vocab
    kv = 0.0
    for t0 in lens:
        for step in range(1, n_new):
            t = t0 + step  # keys of this step
            kv += c.layers * (16.0 * (2 * t * c.d + 2 * c.d) + 8.0 * c.heads * t)
    return weights + kv / (n_new - 1)


def load_traffic(kernel_class, workload):
    """HBM bytes per launch measured by rocprofv3 counters for this class and
    workload (profiles/<class>_<workload>_traffic.json, written by python -m
    rustcrates_amd.traffic), with where it came from.  A measurement whose
    source hash differs from the current sources is stale: traffic is then
    None and the note says so."""
    from rustcrates_amd.build import source_hash

    path = os.path.join(ROOT, "profiles", f"{kernel_class}_{workload}_traffic.json")
    if not os.path.exists(path):
        return None, "no counter measurement for this class and workload"
    with open(path) as fh:
        t = json.load(fh)
    if t.get("kernel_class") != kernel_class or t.get("workload") != workload:
        return None, f"{os.path.basename(path)} is for another class or workload"
    sha = source_hash()
    if t.get("csrc_sha") != sha:
        return None, f"{os.path.basename(path)} measured on sources {t.get('csrc_sha')}, now {sha}: stale"
    return round(t["traffic_bytes_per_launch"], 1), f"{os.path.basename(path)} (sources {sha})"


def roofline_entry(r, bound):
    """Achieved rate of a kernel class from its HIP-event totals (each launch's
    start and stop stamped by its dispatch on the library's stream)."""
    n = max(r["launches"], 1)
    avg_s = r["total_ms"] / n / 1e3
    if bound == "hbm":
        achieved = r["alg_bytes"] / n / avg_s / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    else:
        achieved = r["alg_flops"] / n / avg_s / 1e12
        peak, unit = FP64_MFMA_PEAK_TFS, "TFLOP/s"
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": None, "avg_launch_us": round(avg_s * 1e6, 3),
            "launches": r["launches"], "alg_bytes_per_launch": r["alg_bytes"] / n,
            "alg_flops_per_launch": r["alg_flops"] / n}


def host_threads():
    """CPU threads this process may use: the OMP_NUM_THREADS the host sets for
    it (the GPU box allots 16 per GPU), else every CPU in its affinity mask."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


def cpu_baseline(w, budget_s=20.0):
    """The CPU oracle (a port of the reference's forward, OpenMP over the
    reference's rayon axes) on the first sequences of the same workload."""
    import oracle

    threads = host_threads()
    oracle.set_threads(threads)
    cfg = w.model
    o = configs.build_network(oracle.Network(), cfg)
    prompt, lens = workload_prompt(w)
    nseq, n_new = 1, w.n_new
    t0 = time.perf_counter()
    o.generate(prompt[:1], lens=lens[:1], n_new=n_new)
    t1 = time.perf_counter() - t0
    if t1 < budget_s / 3 and w.batch > 1:
        nseq = int(min(w.batch, max(1, budget_s // max(t1, 1e-3))))
        t0 = time.perf_counter()
        o.generate(prompt[:nseq], lens=lens[:nseq], n_new=n_new)
        t1 = time.perf_counter() - t0
    o.close()
    return {"value": round(nseq * n_new / t1, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "host_cpus": os.cpu_count(),
            "sample": f"{nseq} of {w.batch} sequences, full prompt + {n_new} greedy tokens, {t1:.1f} s, "
                      f"{threads} OpenMP threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="c3b32", choices=sorted(configs.WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-b1", action="store_true", help="skip the batch-1 companion measurement")
    ap.add_argument("--no-train", action="store_true", help="skip the output-head training-step measurement")
    ap.add_argument("--no-classes", action="store_true",
                    help="skip the per-kernel-class HIP-event pass (profiler runs of the timed region only)")
    ap.add_argument("--direct", action="store_true",
                    help="launch decode kernels directly instead of replaying HIP graphs (for profilers)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(sequences shard data-parallel with no exchange; only the one-GPU share is built)", file=sys.stderr)
        sys.exit(2)

    w = configs.WORKLOADS[args.workload]
    log(f"workload {args.workload}: building seeded network")
    with ra.Network(0) as net:
        out = run(args, w, configs.build_network(net, w.model))
    # the network is released before the CPU baseline and before interpreter exit
    if not args.no_cpu:
        log("cpu baseline (oracle)")
        out["cpu_baseline"] = cpu_baseline(w)
    print(json.dumps(out), flush=True)


def run(args, w, net):
    cfg = w.model
    net.set_graph_mode(args.direct)
    prompt, lens = workload_prompt(w)
    B, n_new = w.batch, w.n_new

    log(f"timing {args.steps} steps after {args.warmup} warmup")
    wall, pre_ms, dec_ms, _ = time_generate(net, prompt, lens, n_new, args.steps, args.warmup)
    ms_step = wall / args.steps * 1e3
    tokens = B * n_new
    value = tokens * args.steps / wall
    decode_tok_s = B * (n_new - 1) / (dec_ms / 1e3) if dec_ms > 0 else None

    # roofline of the dominant kernel classes, HIP events on the library stream
    roof, class_ms, prefill_gemm_roof, class_roofs = None, None, None, None
    if not args.no_classes:
        log("kernel-class timing")
        classes = {}
        for name, cls in (("vocab", ra.TIME_VOCAB), ("layer_gemm", ra.TIME_LAYER_GEMM),
                          ("attention", ra.TIME_ATTENTION), ("prefill_gemm", ra.TIME_PREFILL_GEMM)):
            classes[name] = kernel_class(net, prompt, lens, n_new, cls)
        # the dominant class of the decode step (the prompt pass has its own
        # entry below); a class is MFMA-bound when its arithmetic intensity
        # exceeds the ridge point, else HBM-bound
        ridge = FP64_MFMA_PEAK_TFS * 1e12 / (HBM_PEAK_GBS * 1e9)
        class_roofs = {}
        for k in ("vocab", "layer_gemm", "attention"):
            r = classes[k]
            if not r["launches"]:
                continue
            intensity = r["alg_flops"] / max(r["alg_bytes"], 1.0)
            e = roofline_entry(r, "mfma" if intensity > ridge else "hbm")
            e["kernel_class"] = k
            class_roofs[k] = e
        dominant = max(class_roofs, key=lambda k: classes[k]["total_ms"])
        roof = dict(class_roofs[dominant])
        roof["traffic"], roof["traffic_source"] = load_traffic(dominant, args.workload)
        class_ms = {k: round(v["total_ms"] / 2, 3) for k, v in classes.items()}
        prefill_gemm_roof = (roofline_entry(classes["prefill_gemm"], "mfma")
                             if classes["prefill_gemm"]["launches"] else None)

    out = {
        "metric": "generated tokens/s",
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "c128",
        "data": "synthetic (seeded Xavier-uniform weights, uniform-random prompt ids)",
        "config": {"workload": args.workload, "layers": cfg.layers, "d_model": cfg.d, "heads": cfg.heads,
                   "ffn": cfg.ffn, "vocab": cfg.vocab, "batch": B, "prompt_len": w.prompt_len,
                   "n_new": n_new, "parallelism": "single GPU"},
        "prefill_ms": round(pre_ms, 3),
        "decode_ms": round(dec_ms, 3),
        "decode_tokens_per_s": round(decode_tok_s, 2) if decode_tok_s else None,
        "kernel_class_ms_per_step": class_ms,
        "roofline": roof,
        "class_rooflines": ({k: {"bound": v["bound"], "achieved": v["achieved"], "unit": v["unit"],
                                 "frac": v["frac"], "avg_launch_us": v["avg_launch_us"]}
                             for k, v in class_roofs.items()} if class_roofs else None),
    }
    # the prompt pass against the FP64 MFMA peak (north_star's prefill target)
    pf = prefill_flops(w, [int(x) for x in lens])
    out["prefill"] = {
        "alg_gflop": round(pf / 1e9, 2),
        "tflops": round(pf / (pre_ms / 1e3) / 1e12, 3),
        "mfma_frac": round(pf / (pre_ms / 1e3) / 1e12 / FP64_MFMA_PEAK_TFS, 4),
        "gemm_roofline": prefill_gemm_roof,
    }
    # the whole decode step against the HBM roofline: every weight once plus
    # each sequence's KV rows and bias row 0 (the step's algorithmic bytes)
    sb = decode_step_bytes(cfg, [int(x) for x in lens], n_new)
    out["decode_step_bytes"] = round(sb)
    out["decode_step_hbm_frac"] = round(sb / (dec_ms / (n_new - 1) / 1e3) / 1e9 / HBM_PEAK_GBS, 4)

    if not args.no_b1 and B > 1 and args.workload.startswith("c3"):
        log("batch-1 companion")
        w1 = configs.WORKLOADS["c3b1"]
        p1, l1 = workload_prompt(w1)
        wall1, pre1, dec1, _ = time_generate(net, p1, l1, w1.n_new, max(3, args.steps), 1)
        rv = kernel_class(net, p1, l1, w1.n_new, ra.TIME_VOCAB)
        out["batch1"] = {
            "tokens_per_s": round(w1.n_new * max(3, args.steps) / wall1, 2),
            "decode_tokens_per_s": round((w1.n_new - 1) / (dec1 / 1e3), 2),
            "decode_ms_per_token": round(dec1 / (w1.n_new - 1), 4),
            "prefill_ms": round(pre1, 3),
            "vocab_roofline": roofline_entry(rv, "hbm"),
        }
        # whole decode step against the HBM roofline: weights + KV + bias rows per token
        step_bytes = decode_step_bytes(cfg, [int(x) for x in l1], w1.n_new)
        out["batch1"]["decode_step_bytes"] = round(step_bytes)
        out["batch1"]["decode_step_hbm_frac"] = round(step_bytes / (dec1 / (w1.n_new - 1) / 1e3) / 1e9 / HBM_PEAK_GBS, 4)

    if not args.no_train and args.workload.startswith("c3"):
        log("output-head training step")
        out["head_train"] = head_train_step(cfg)
        out["train_step"] = train_step(cfg)

    return out


def head_train_step(cfg, B=8, S=128, T=64, reps=5):
    """The output head's training step (mitok_backward_head: Softmax
    cross-entropy gradient, vocab Linear backward, then its AdamW update) at
    config 3's head shapes, after one TRAINING-mode predict of B x S rows.
    Algorithmic flops: the two products dW = conj(X)^T G and dX = G conj(W)^T,
    8 * d * V * rows each."""
    with ra.Network(0) as h:
        h.add_embedding(cfg.vocab, cfg.d)
        h.add_linear(cfg.d, cfg.vocab)
        h.add_softmax(ra.TRAINING)
        h.init_seeded(cfg.seed)
        ids = seeded.prompts(11, [S] * B, cfg.vocab)
        targets = seeded.prompts(12, [T] * B, cfg.vocab)
        h.predict(ids, forward_only=False)
        for t in (1, 2):  # the first update (plain descent), then AdamW
            h.backward_head(targets, update=True, learning_rate=1e-3, time_step=t, want_grad_input=False)
        ra.device_synchronize(0)
        t0 = time.perf_counter()
        for t in range(reps):
            h.backward_head(targets, update=True, learning_rate=1e-3, time_step=3 + t, want_grad_input=False)
        ms = (time.perf_counter() - t0) / reps * 1e3
    flops = 2 * 8.0 * cfg.d * cfg.vocab * B * S
    return {"config": f"vocab Linear {cfg.d} x {cfg.vocab}, {B} x {S} rows, {T} targets per sequence, AdamW update",
            "ms_per_step": round(ms, 3), "alg_gflop": round(flops / 1e9, 2),
            "tflops": round(flops / (ms / 1e3) / 1e12, 3),
            "mfma_frac": round(flops / (ms / 1e3) / 1e12 / FP64_MFMA_PEAK_TFS, 4)}


def train_step(cfg, B=8, S=128, T=64, reps=3):
    """One step of the reference's train loop (transformer_network.rs:35-163)
    on config 3: the TRAINING-mode predict of B x S rows and
    cross_entropy_loss_batch on its softmax output, both on the device (only
    the loss crosses PCIe, mitok_cross_entropy_loss), then backward over every
    layer with every update (mitok_backward).  Algorithmic flops of the
    backward's products (8 M N K each): per attention layer the Q/K/V
    recompute, their weight and input gradients (3 x 24 rows d^2); per
    FeedForward the Dense recompute twice and four gradient products
    (6 x 8 rows d F); the vocab Linear's two (16 rows d V)."""
    rows = B * S
    with ra.Network(0) as net:
        configs.build_network(net, cfg, mode=ra.TRAINING)
        ids = seeded.prompts(21, [S] * B, cfg.vocab)
        targets = seeded.prompts(22, [T] * B, cfg.vocab)
        nl = net.num_layers
        for t in (1, 2):  # every layer's first update (plain descent), then AdamW
            net.predict(ids, forward_only=False, want_output=False)
            net.cross_entropy_loss(targets)
            net.backward(targets, layers=nl - 1, update=True, learning_rate=1e-4, time_step=t, want_grad_input=False)
        ra.device_synchronize(0)
        fwd = bwd = 0.0
        losses = []
        for t in range(reps):
            t0 = time.perf_counter()
            net.predict(ids, forward_only=False, want_output=False)
            losses.append(net.cross_entropy_loss(targets).real)
            t1 = time.perf_counter()
            net.backward(targets, layers=nl - 1, update=True, learning_rate=1e-4, time_step=3 + t, want_grad_input=False)
            fwd += t1 - t0
            bwd += time.perf_counter() - t1
    fwd_ms, bwd_ms = fwd / reps * 1e3, bwd / reps * 1e3
    d, F, V = cfg.d, cfg.ffn, cfg.vocab
    flops = cfg.layers * (3 * 24.0 * rows * d * d + 6 * 8.0 * rows * d * F) + 16.0 * rows * d * V
    return {"config": f"{cfg.name}, {B} x {S} rows, {T} targets per sequence, backward over all {nl - 1} "
                      "layers below the Softmax with every update",
            "forward_ms": round(fwd_ms, 3), "backward_ms": round(bwd_ms, 3),
            "loss": [round(x, 6) for x in losses],
            "backward_alg_gflop": round(flops / 1e9, 2),
            "backward_tflops": round(flops / (bwd_ms / 1e3) / 1e12, 3)}


if __name__ == "__main__":
    main()
