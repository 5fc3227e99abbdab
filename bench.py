"""Benchmark: 12-layer GPT decoder prefill on the MI355X HIP engine.

BASELINE.json metric "decoder inference tokens/s at 1 GPU" on configs[4]
(GPT-style decoder bf16: 12 layers, d_model 768, 12 heads, FFN 3072 GELU,
vocab 32000, causal, batch 4, seq 1024, full prefill forward to logits),
with seeded uniform token ids and N(0, 0.02) weights.

One step = one compiled forward (one hipGraph launch) over the resident
[4, 1024] ids already in HBM.  W untimed warm-up steps, then exactly K timed
steps bracketed by torch.cuda.synchronize() on both sides.

Roofline: every op of the compiled forward is also timed on its own with
HIP events on the engine stream it runs on (mh_engine_op_times: 20 launches
of the op captured in one graph and replayed between events, so host launch
cost is excluded; the rocprofv3 kernel trace of the same command shows the
same per-dispatch durations); the kernel with the largest time per forward
is reported against the bf16 MFMA peak (GEMM / attention: algorithmic
2*M*N*K FLOPs) or the HBM peak (LayerNorm: unique bytes), and against the measured peaks (the
register-only MFMA loop of mh_measure_mfma_peak; a 1 GiB device copy).
Inside the
forward the kernels run with colder caches: "kernels_in_forward_avg_us"
(mh_engine_forward_op_times: differences of prefix-graph times, each over 20
replays; an op's figure also carries what it costs the ops after it, such as
the write-back of its output, and the first op carries the graph launch).
CPU baseline: the C++ restatement
of MuNet's CPU backend (oracle/, "port") on a bounded sample of the same
forward, timed on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16 = 2.5e15      # dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12       # HBM3E, B/s

CFG = dict(vocab=32000, ctx=1024, d_model=768, num_heads=12, num_layers=12, ffn=3072, dtype="bfloat16")
B, T = 4, 1024


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ops of the compiled forward grouped into the kernels of the roofline table
def op_category(op):
    name, kind = op["name"], op["kind"]
    if kind == "qkv_gemm":
        return "qkv_headsplit"
    if kind == "attention":
        return "attention_causal"
    if kind == "layer_norm":
        return "layer_norm"
    if kind.startswith("embedding"):
        return "embedding"
    if name.endswith("out_proj"):
        return "attn_out_resid"
    if ".ff.0" in name:
        return "ffn_up_gelu"
    if ".ff.2" in name:
        return "ffn_down_resid"
    if name.startswith("head"):
        return "lm_head"
    return name


def kernel_table(eng, reps=20, in_forward=True):
    """Per-kernel timing of the compiled forward's own ops (the LayerNorm-
    folded consumers and the statistics-producing residual GEMMs as the
    forward runs them).  in_forward: mh_engine_forward_op_times, differences
    of prefix-graph times, each over `reps` replays (the forward's own caches
    and transitions); otherwise mh_engine_op_times, each op replayed `reps`
    times from one graph (warm caches).  Rows: one per kernel
    category with the mean time per launch, launches per forward and
    algorithmic work per launch."""
    cats = {}
    for op in (eng.forward_op_times(reps) if in_forward else eng.op_times(reps)):
        c = cats.setdefault(op_category(op), dict(ts=[], flops=op["flops"], bytes=op["bytes"], first=op["name"]))
        c["ts"].append(op["us"] * 1e-6)
    return [dict(name=n, t=sum(c["ts"]) / len(c["ts"]), count=len(c["ts"]), flops=c["flops"], bytes=c["bytes"],
                 op=c["first"]) for n, c in cats.items()]


COPY_BYTES = 256 << 20  # the calibration copy of --probe


def probe(eng, torch, name):
    """For rocprofv3 --pmc passes: one forward, then 5 replayed launches of
    the first op of category `name` (mh_engine_op_times restricted to that
    op), then one device-to-device copy of COPY_BYTES (the counter
    calibration: it reads and writes exactly that many bytes)."""
    op = next(r["op"] for r in kernel_table(eng, 1, in_forward=False) if r["name"] == name)
    torch.cuda.synchronize()
    eng.op_times(5, only=op)
    torch.cuda.synchronize()
    a = torch.ones(COPY_BYTES // 2, device="cuda", dtype=torch.bfloat16)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    log(f"probe: {name} ({op}) x5 after a forward, copy {COPY_BYTES} bytes")


def measured_traffic(name):
    """HBM bytes per launch of `name` from its committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/<name>_traffic.md), or None."""
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline():
    """Oracle restatement on a bounded sample: 1 of the 12 decoder layers plus
    final LayerNorm + LM head for 1 of the 4 sequences (1024 tokens), the
    forward time extrapolated to 12 layers."""
    from munet_amd import models, synth
    from oracle import CpuOracle
    from oracle import models as om
    orc = CpuOracle("restatement")
    cfg = models.decoder_config(**{**CFG, "num_layers": 1})
    params = models.init_params(cfg, "gpt", scope="cpu")
    ids = models.make_input(cfg, (1, T), "gpt", scope="cpu_in")
    dt = synth.BF16
    t0 = time.perf_counter()
    x = om.decoder_embed(orc, cfg, params, ids)
    t1 = time.perf_counter()
    x = om.block_forward(orc, cfg, params, x, "blocks.0.", True)
    t2 = time.perf_counter()
    x = orc.layer_norm(x, params["ln_f.weight"], params["ln_f.bias"], dt)
    orc.linear(x, params["head.weight"], params["head.bias"], dt)
    t3 = time.perf_counter()
    fwd = (t1 - t0) + CFG["num_layers"] * (t2 - t1) + (t3 - t2)
    return dict(value=T / fwd, unit="tokens/s", cores=orc.threads(), kind="port",
                sample=(f"1 of 12 decoder layers + ln_f + LM head on 1 sequence x {T} tokens "
                        f"({t3 - t0:.1f} s measured: embed {t1 - t0:.2f}s, layer {t2 - t1:.2f}s, "
                        f"head {t3 - t2:.2f}s), extrapolated to 12 layers"))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--probe", default=None, help="run one kernel of the forward for rocprofv3 --pmc and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the single-GPU design and how the path would shard are in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch
    import ctypes

    from munet_amd import _lib, models
    from munet_amd.engine import Engine

    cfg = models.decoder_config(**CFG)
    log("bench: initialising weights")
    params = models.init_params(cfg, "gpt", scope="bench")
    ids = models.make_input(cfg, (B, T), "gpt", scope="bench_in")
    log("bench: compiling engine")
    eng = Engine(0).load(cfg, params).compile((B, T))
    del params
    logits = eng.run(ids)  # places the ids in the engine's input buffer (HBM)
    assert np.isfinite(logits[:, :8].astype(np.float32)).all()
    if args.probe:
        probe(eng, torch, args.probe)
        return

    for _ in range(args.warmup):
        eng.launch()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.launch()
    torch.cuda.synchronize()
    dt_s = time.perf_counter() - t0
    ms = dt_s / args.steps * 1e3
    tokens_s = B * T * args.steps / dt_s
    log(f"bench: {ms:.3f} ms/forward, {tokens_s:,.0f} tokens/s")
    # the timed forwards reran the resident input: no device error (token id
    # out of range) and the same logits as the first forward, bit for bit
    _lib.call("mh_check_device_errors")
    again = np.empty_like(logits)
    _lib.call("mh_copy", ctypes.c_void_p(eng.output_ptr()), again.ctypes.data_as(ctypes.c_void_p),
              ctypes.c_size_t(again.nbytes), 1, 0, ctypes.c_void_p(eng.stream()))
    if not np.array_equal(again.view(np.uint16), logits.view(np.uint16)):
        raise SystemExit("bench: repeated forwards changed the logits")

    # measured peaks beside the datasheet ones: the MFMA loop of peak.hip,
    # and a 1 GiB device-to-device copy (reads and writes 2 GiB)
    from munet_amd.backend import HipBackend
    peak_mfma = HipBackend(0).measure_mfma_peak(2, 16000)
    src = torch.empty(1 << 29, device="cuda", dtype=torch.float16)
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    peak_hbm = 5 * 2.0 * src.numel() * 2 / (e0.elapsed_time(e1) * 1e-3)
    del src, dst

    rows = kernel_table(eng, in_forward=False)
    # in-forward times are differences of prefix-graph times: a few us of
    # replay-to-replay noise each, so only the per-layer categories (means over
    # 12 ops) and the LM head (hundreds of us) are reported
    fwd = {r["name"]: round(r["t"] * 1e6, 2) for r in kernel_table(eng, in_forward=True)
           if r["count"] >= 12 or r["name"] == "lm_head"}
    for r in rows:
        r["per_fwd"] = r["t"] * r["count"]
    dom = max(rows, key=lambda r: r["per_fwd"])
    if dom["flops"]:
        ach = dom["flops"] / dom["t"]
        roof = dict(bound="mfma", achieved=ach / 1e12, peak=PEAK_BF16 / 1e12, unit="TFLOP/s", frac=ach / PEAK_BF16,
                    peak_measured=peak_mfma / 1e12, frac_of_measured=ach / peak_mfma)
    else:
        ach = dom["bytes"] / dom["t"]
        roof = dict(bound="hbm", achieved=ach / 1e9, peak=PEAK_HBM / 1e9, unit="GB/s", frac=ach / PEAK_HBM,
                    peak_measured=peak_hbm / 1e9, frac_of_measured=ach / peak_hbm)
    roof.update(kernel=dom["name"], avg_us=dom["t"] * 1e6, traffic=measured_traffic(dom["name"]))
    gemm = [r for r in rows if r["flops"] and r["name"] != "attention_causal"]
    gemm_frac = sum(r["flops"] * r["count"] for r in gemm) / sum(r["per_fwd"] for r in gemm) / PEAK_BF16
    ln = next(r for r in rows if r["name"] == "layer_norm")
    kernels = {r["name"]: dict(avg_us=round(r["t"] * 1e6, 2), per_forward=r["count"],
                               tflops=round(r["flops"] / r["t"] / 1e12, 1) if r["flops"] else None,
                               gbs=round(r["bytes"] / r["t"] / 1e9, 1) if r["bytes"] else None) for r in rows}

    cpu = None
    if not args.no_cpu_baseline:
        log("bench: timing the CPU baseline sample")
        cpu = cpu_baseline()
    line = {
        "metric": "decoder inference tokens/s at 1 GPU",
        "value": tokens_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded uniform token ids [4,1024], N(0,0.02) weights (random init)",
        "config": {"workload": "gpt_decoder_prefill (BASELINE configs[4])", "layers": 12, "d_model": 768,
                   "heads": 12, "ffn": 3072, "vocab": 32000, "batch": B, "seq_len": T, "causal": True,
                   "tokens_per_step": B * T},
        "roofline": roof,
        "gemm_mfma_frac": gemm_frac,
        "layernorm_hbm_frac": (ln["bytes"] / ln["t"]) / PEAK_HBM,
        "measured_peaks": {"mfma_bf16_tflops": peak_mfma / 1e12, "hbm_copy_gbs": peak_hbm / 1e9},
        "kernels": kernels,
        "kernels_in_forward_avg_us": fwd,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
