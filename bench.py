"""Benchmark: 12-layer GPT decoder prefill on the MI355X HIP engine, plus the
other BASELINE workloads.

Headline (BASELINE.json metric "decoder inference tokens/s at 1 GPU",
configs[4]): GPT-style decoder bf16, 12 layers, d_model 768, 12 heads, FFN
3072 GELU, vocab 32000, causal, batch 4, seq 1024, full prefill forward to
logits, with seeded uniform token ids and N(0, 0.02) weights.  One step = one
compiled forward (one hipGraph launch) over the resident [4, 1024] ids already
in HBM.  W untimed warm-up steps, then exactly K timed steps bracketed by
torch.cuda.synchronize() on both sides.

Roofline: every op's cost inside the forward is measured with HIP events on
the engine stream as differences of prefix-graph times (for each prefix
ops[0..i] of the forward, 20 back-to-back replays between two events; op i's
cost is T(i) - T(i-1), which also holds what it costs the ops after it,
mh_engine_forward_op_times).  The kernel category with the largest cost per
forward is the dominant one.  Its launch duration is timed with HIP events
over 20 back-to-back launches of the forward's own op (the same arena
buffers, the folded-LayerNorm and statistics programs) replayed from one
graph on the engine stream (mh_engine_op_times; these are dispatches a
kernel trace of the same command shows), and its algorithmic work per
launch (GEMM 2*M*N*K FLOPs, causal attention 4*B*H*T^2*hd/2, LayerNorm
unique bytes) over that duration is `achieved`, against the datasheet peak
and against the measured ones (the register-only MFMA loop of
mh_measure_mfma_peak; a read-only stream over 2 GiB, mh_measure_hbm_read; a
1 GiB device copy).

CPU baseline: MuNet's own CPU code (oracle/_ref: the reference sources
compiled by oracle/Makefile, kind "reference") on a bounded sample of the
same forward on this host, with the C++ restatement of MuNet's CPU backend
(oracle/, kind "port", in its reference-threading mode: CPUBackend::
parallel_for inline below 1024 iterations, the fp16/bf16 fallbacks,
LayerNorm and gathers serial) beside it as a second figure; the port alone
where oracle/_ref is absent or MuNet cannot run the model (the UNet).  One
bf16 Linear is also timed in both ("reference_check").

"configs": BASELINE configs[0..3] (MLP, CNN, encoder block bf16 / fp16,
UNet) at their full sizes: forward time, samples/s, MFMA / HBM fractions of
their products and norms, and the CPU baseline per config; "decode": greedy
KV-cache decode on the headline architecture with textbook-key attention
(ms per step, tokens/s, HBM bytes per step against the 8 TB/s peak).
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

PEAK_BF16 = 2.5e15      # dense bf16 / fp16 MFMA, FLOP/s
PEAK_F32 = 157.3e12     # fp32 MFMA, FLOP/s
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


def categorise(ops):
    """Rows per kernel category: mean time per launch, launches per forward,
    algorithmic work per launch, the op names."""
    cats = {}
    for op in ops:
        c = cats.setdefault(op_category(op), dict(ts=[], flops=op["flops"], bytes=op["bytes"], names=[]))
        c["ts"].append(op["us"] * 1e-6)
        c["names"].append(op["name"])
    return {n: dict(name=n, t=sum(c["ts"]) / len(c["ts"]), count=len(c["ts"]), flops=c["flops"], bytes=c["bytes"],
                    names=c["names"]) for n, c in cats.items()}


COPY_BYTES = 256 << 20  # the calibration copy of --probe


def probe(eng, torch, name):
    """For rocprofv3 --pmc passes: one forward, then 5 replayed launches of
    the first op of category `name` (mh_engine_op_times restricted to that
    op), then one device-to-device copy of COPY_BYTES (the counter
    calibration: it reads and writes exactly that many bytes)."""
    op = categorise(eng.op_times(1))[name]["names"][0]
    torch.cuda.synchronize()
    eng.op_times(5, only=op)
    torch.cuda.synchronize()
    a = torch.ones(COPY_BYTES // 2, device="cuda", dtype=torch.bfloat16)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    log(f"probe: {name} ({op}) x5 after a forward, copy {COPY_BYTES} bytes")


def probe_config(torch, key, op):
    """--probe for a BASELINE config (--config KEY --probe OP, OP an op name
    of its plan): one forward, then 5 replayed launches of that op, then the
    calibration copy, as probe() does for the decoder."""
    from munet_amd import models
    from munet_amd.engine import Engine
    w = models.baseline_workloads()[key]
    cfg, shape, init = w["config"], w["input_shape"], w["init"]
    eng = Engine(0).load(cfg, models.init_params(cfg, init, scope=f"bench_{key}")).compile(shape)
    eng.run(models.make_input(cfg, shape, init, scope=f"bench_{key}_in"))
    names = [o["name"] for o in eng.plan()["ops"]]
    if op not in names:
        sys.exit(f"bench: no op {op!r} in the {key} plan (one of {names})")
    torch.cuda.synchronize()
    eng.op_times(5, only=op)
    torch.cuda.synchronize()
    a = torch.ones(COPY_BYTES // 2, device="cuda", dtype=torch.bfloat16)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    log(f"probe: {key} {op} x5 after a forward, copy {COPY_BYTES} bytes")
    eng.close()


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


def timed_launches(eng, torch, steps, warmup):
    for _ in range(warmup):
        eng.launch()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.launch()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


# ---- CPU baseline ------------------------------------------------------------

def _timed(fn):
    t0 = time.perf_counter()
    out = fn()
    return out, time.perf_counter() - t0


def reference_check():
    """One bf16 Linear (16 x 768 -> 3072) in MuNet's own compiled CPU code
    (oracle/_ref) and in the port's reference-threading mode, when oracle/_ref
    is present: the port's bf16 fallback is leaner than MuNet's per-element
    ScalarValue reads, so its times understate MuNet's."""
    from munet_amd import synth
    from oracle import CpuOracle, available
    if not available("reference"):
        return None
    ref, port = CpuOracle("reference"), CpuOracle("restatement")
    port.set_threading("reference")
    rng = np.random.default_rng(7)
    dt = synth.BF16
    x = synth.encode(rng.standard_normal((16, 768)), dt)
    w = synth.encode(rng.standard_normal((768, 3072)) * 0.02, dt)
    b = synth.encode(np.zeros(3072), dt)
    y_ref, t_ref = _timed(lambda: ref.linear(x, w, b, dt))
    y_port, t_port = _timed(lambda: port.linear(x, w, b, dt))
    port.set_threading("parity")
    return dict(op="bf16 Linear 16x768 -> 3072", munet_s=round(t_ref, 4), port_s=round(t_port, 4),
                munet_over_port=round(t_ref / t_port, 3), same_bits=bool(np.array_equal(y_ref, y_port)))


_GPT_SAMPLE = {}


def gpt_cpu_sample():
    """The one-layer decoder (headline dimensions), its seeded parameters and
    one 1024-token sequence, shared by both CPU baselines (generating the
    parameters takes seconds)."""
    if not _GPT_SAMPLE:
        from munet_amd import models
        cfg = models.decoder_config(**{**CFG, "num_layers": 1})
        _GPT_SAMPLE.update(cfg=cfg, p=models.init_params(cfg, "gpt", scope="cpu"),
                           ids=models.make_input(cfg, (1, T), "gpt", scope="cpu_in"))
    return _GPT_SAMPLE["cfg"], _GPT_SAMPLE["p"], _GPT_SAMPLE["ids"]


def cpu_baseline_gpt(rows=32):
    """Port in reference-threading mode on one 1024-token sequence: the row-
    wise ops of one decoder layer (embedding, LayerNorms, residual adds) on all
    1024 rows, its Linears and GELU on `rows` rows scaled to 1024, attention
    (per (b, h) block: a lower bound on MuNet's dense [B*H*T]^2 path) on all
    rows; the layer time x 12 plus ln_f and the LM head (on `rows` rows,
    scaled).  In MuNet every one of these bf16 ops is a serial fallback."""
    from munet_amd import synth
    from oracle import CpuOracle
    from oracle import models as om
    orc = CpuOracle("restatement")
    cfg, p, ids = gpt_cpu_sample()
    dt, d, H, pre = synth.BF16, CFG["d_model"], CFG["num_heads"], "blocks.0."
    scale = T / rows
    lin = lambda x, n: orc.linear(x, p[n + ".weight"], p[n + ".bias"], dt)  # noqa: E731
    tm = {}
    orc.set_threading("reference")
    try:
        x, tm["embed"] = _timed(lambda: om.decoder_embed(orc, cfg, p, ids).reshape(T, d))
        h, tm["ln1"] = _timed(lambda: orc.layer_norm(x, p[pre + "ln1.weight"], p[pre + "ln1.bias"], dt))
        tm["qkv"] = sum(_timed(lambda n=n: lin(h[:rows], pre + "attn." + n))[1] for n in ("q_proj", "k_proj", "v_proj"))
        orc.set_threading("parity")  # full q / k / v for the attention, untimed
        q, k, v = (lin(h, pre + "attn." + n) for n in ("q_proj", "k_proj", "v_proj"))
        orc.set_threading("reference")
        ctx, tm["attention"] = _timed(lambda: orc.mha_core(q, k, v, 1, T, H, True, dt))
        a, tm["out_proj"] = _timed(lambda: lin(ctx[:rows], pre + "attn.out_proj"))
        x2, tm["residual1"] = _timed(lambda: orc.add(x, np.resize(a, x.shape), dt))
        h2, tm["ln2"] = _timed(lambda: orc.layer_norm(x2, p[pre + "ln2.weight"], p[pre + "ln2.bias"], dt))
        f, tm["ffn_up"] = _timed(lambda: lin(h2[:rows], pre + "ff.0"))
        g, tm["gelu"] = _timed(lambda: orc.gelu(f, dt))
        f2, tm["ffn_down"] = _timed(lambda: lin(g, pre + "ff.2"))
        _, tm["residual2"] = _timed(lambda: orc.add(x2, np.resize(f2, x2.shape), dt))
        hf, tm["ln_f"] = _timed(lambda: orc.layer_norm(x2, p["ln_f.weight"], p["ln_f.bias"], dt))
        _, tm["head"] = _timed(lambda: lin(hf[:rows], "head"))
    finally:
        orc.set_threading("parity")
    sampled = ("qkv", "out_proj", "ffn_up", "gelu", "ffn_down", "head")
    full = {k: v * (scale if k in sampled else 1.0) for k, v in tm.items()}
    layer = sum(v for k, v in full.items() if k not in ("embed", "ln_f", "head"))
    fwd = full["embed"] + CFG["num_layers"] * layer + full["ln_f"] + full["head"]
    measured = sum(tm.values())
    return dict(value=T / fwd, unit="tokens/s", cores=1, kind="port",
                threading="reference (every bf16 op of this model is a serial fallback in MuNet)",
                host_threads=orc.threads(), cpu_model=cpu_model(),
                sample=(f"one 1024-token sequence through one decoder layer: Linears, GELU and the LM head on "
                        f"{rows} rows scaled x{scale:.0f}, row-wise ops and per-block attention on all rows "
                        f"({measured:.1f} s measured: layer {layer:.2f} s, head {full['head']:.2f} s as extrapolated), "
                        f"extrapolated to 12 layers; per-block attention is a lower bound on MuNet's dense "
                        f"[B*H*T]^2 attention"),
                seconds_per_forward_of_one_sequence=fwd)


def cpu_reference_gpt(rows=32, t_fit=(64, 128)):
    """MuNet's own compiled CPU code (oracle/_ref: the reference sources built
    by oracle/Makefile, the ops driven through ref_driver.cpp) on one
    1024-token sequence, the same sample as the port's: the row-wise ops of
    one decoder layer on all 1024 rows, its Linears and GELU on `rows` rows
    scaled to 1024, the layer x 12 plus ln_f and the LM head (`rows` rows,
    scaled).  nn::MultiHeadAttention is MuNet's dense path (the [H*T]^2 mask,
    masked_fill, softmax and both products over every head pair): its time
    is a*T + c*T^2 (projections linear in T, the rest quadratic), measured
    on the first t_fit[0] and t_fit[1] tokens of the same layer, solved for
    a and c and evaluated at T = 1024.  Every bf16 op here is one of MuNet's
    serial fallbacks (one core)."""
    from munet_amd import synth
    from oracle import CpuOracle, available
    from oracle import models as om
    if not available("reference"):
        return None
    ref = CpuOracle("reference")
    cfg, p, ids = gpt_cpu_sample()
    dt, d, H, pre = synth.BF16, CFG["d_model"], CFG["num_heads"], "blocks.0."
    scale = T / rows
    lin = lambda x, n: ref.linear(x, p[n + ".weight"], p[n + ".bias"], dt)  # noqa: E731
    tm = {}
    x, tm["embed"] = _timed(lambda: om.decoder_embed(ref, cfg, p, ids).reshape(T, d))
    h, tm["ln1"] = _timed(lambda: ref.layer_norm(x, p[pre + "ln1.weight"], p[pre + "ln1.bias"], dt))
    (t1, t2), ts = t_fit, []
    for tt in (t1, t2):
        ts.append(_timed(lambda tt=tt: ref.mha(h[None, :tt], p, H, True, dt, prefix=pre + "attn."))[1])
    c = (ts[1] - ts[0] * t2 / t1) / (t2 * t2 - t1 * t2)
    a = (ts[0] - c * t1 * t1) / t1
    mha_t = a * T + c * T * T
    x2, tm["residual1"] = _timed(lambda: ref.add(x, h, dt))  # the add's cost does not depend on the values
    h2, tm["ln2"] = _timed(lambda: ref.layer_norm(x2, p[pre + "ln2.weight"], p[pre + "ln2.bias"], dt))
    f, tm["ffn_up"] = _timed(lambda: lin(h2[:rows], pre + "ff.0"))
    g, tm["gelu"] = _timed(lambda: ref.gelu(f, dt))
    f2, tm["ffn_down"] = _timed(lambda: lin(g, pre + "ff.2"))
    _, tm["residual2"] = _timed(lambda: ref.add(x2, np.resize(f2, x2.shape), dt))
    hf, tm["ln_f"] = _timed(lambda: ref.layer_norm(x2, p["ln_f.weight"], p["ln_f.bias"], dt))
    _, tm["head"] = _timed(lambda: lin(hf[:rows], "head"))
    sampled = ("ffn_up", "gelu", "ffn_down", "head")
    full = {k: v * (scale if k in sampled else 1.0) for k, v in tm.items()}
    full["attention"] = mha_t
    layer = sum(v for k, v in full.items() if k not in ("embed", "ln_f", "head"))
    fwd = full["embed"] + CFG["num_layers"] * layer + full["ln_f"] + full["head"]
    measured = sum(tm.values()) + sum(ts)
    return dict(value=T / fwd, unit="tokens/s", cores=1, kind="reference",
                threading="MuNet's own CPU backend (every bf16 op of this model is one of its serial fallbacks)",
                host_threads=ref_threads(), cpu_model=cpu_model(),
                sample=(f"MuNet's compiled CPU code on one 1024-token sequence through one decoder layer: "
                        f"nn::MultiHeadAttention (dense mask) timed on {t1} and {t2} tokens "
                        f"({ts[0]:.2f} s, {ts[1]:.2f} s) and fitted as a*T + c*T^2 to T = 1024 "
                        f"({mha_t:.1f} s), Linears, GELU and the LM head on {rows} rows scaled x{scale:.0f}, "
                        f"row-wise ops on all rows ({measured:.1f} s measured: layer {layer:.1f} s, head "
                        f"{full['head']:.1f} s as extrapolated), extrapolated to 12 layers"),
                seconds_per_forward_of_one_sequence=fwd)


def ref_threads():
    return os.cpu_count() or 1


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_reference_forward(cfg, params, x):
    """Whole-forward time of MuNet's own compiled CPU code (oracle/_ref) on
    `x`, the model composed from its ops as the oracle composes it, or None
    when oracle/_ref is absent or MuNet cannot run the model (the UNet's
    ConvTranspose2d and 16-bit concat have no MuNet CPU path)."""
    from oracle import CpuOracle, available
    from oracle import models as om
    if not available("reference") or cfg["type"] == "UNet":
        return None
    ref = CpuOracle("reference")
    _, t = _timed(lambda: om.forward(ref, cfg, params, x))
    return t


def cpu_port_forward(cfg, params, x, threading):
    """Whole-forward time of the port on `x` (a bounded sample) in the given
    threading mode."""
    from oracle import CpuOracle
    from oracle import models as om
    orc = CpuOracle("restatement")
    orc.set_threading(threading)
    try:
        _, t = _timed(lambda: om.forward(orc, cfg, params, x))
    finally:
        orc.set_threading("parity")
    return t


# ---- the other BASELINE configs ---------------------------------------------

CONFIG_ROWS = [
    # key, BASELINE index, sample batch for the CPU baseline
    ("mlp", 0, None),
    ("cnn", 1, None),
    ("encoder_bf16", 2, 1),
    ("encoder_fp16", 2, 1),
    ("unet", 3, 1),
]


def config_line(torch, key, idx, cpu_batch, steps, warmup, with_cpu):
    from munet_amd import models, synth
    from munet_amd.engine import Engine
    w = models.baseline_workloads()[key]
    cfg, shape, init = w["config"], w["input_shape"], w["init"]
    dt = synth.DTYPE_CODES[cfg.get("dtype", "float32")]
    params = models.init_params(cfg, init, scope=f"bench_{key}")
    x = models.make_input(cfg, shape, init, scope=f"bench_{key}_in")
    eng = Engine(0).load(cfg, params).compile(shape)
    eng.run(x)
    # a forward here takes 15-600 us: at least 50 untimed and 200 timed
    # back-to-back graph launches, so that the host's launch path is warm
    # (the first few dozen hipGraphLaunch calls of a process cost twice the
    # later ones) and the figure is the steady launch rate
    steps, warmup = max(steps, 200), max(warmup, 50)
    s = timed_launches(eng, torch, steps, warmup)
    ops = eng.op_times(10)
    peak = PEAK_F32 if dt == synth.F32 else PEAK_BF16
    mm = [o for o in ops if o["flops"]]
    mm_t = sum(o["us"] for o in mm) * 1e-6
    mm_f = sum(o["flops"] for o in mm)
    ln = [o for o in ops if o["kind"] == "layer_norm"]
    batch = shape[0]
    row = dict(baseline_config=idx, dtype=synth.DTYPE_NAMES[dt], input_shape=list(shape), ms=s * 1e3,
               timed_launches=steps, warmup_launches=warmup, samples_per_s=batch / s,
               mfma_frac=(mm_f / mm_t / peak) if mm_t else None,
               mfma_tflops=(mm_f / mm_t / 1e12) if mm_t else None,
               mfma_share_of_forward=mm_t / s,
               peak_tflops=peak / 1e12,
               layernorm_hbm_frac=(sum(o["bytes"] for o in ln) / (sum(o["us"] for o in ln) * 1e-6) / PEAK_HBM)
               if ln else None,
               ops=len(ops))
    if key.startswith("encoder"):
        row["tokens_per_s"] = shape[0] * shape[1] / s
    if with_cpu:
        n = cpu_batch or batch
        xs = np.ascontiguousarray(x[:n])
        sample = f"batch {n} of {batch}" + (" (samples are independent)" if n < batch else "")
        t_port = cpu_port_forward(cfg, params, xs, "reference")
        port = dict(value=n / t_port, unit="samples/s", kind="port", threading="reference", sample=sample,
                    seconds=t_port)
        t_munet = cpu_reference_forward(cfg, params, xs)
        if t_munet is not None:
            row["cpu_baseline"] = dict(value=n / t_munet, unit="samples/s", kind="reference",
                                       threading="MuNet's own CPU backend", host_threads=ref_threads(),
                                       sample=sample, seconds=t_munet, port=port)
        else:
            row["cpu_baseline"] = dict(port, note="MuNet's CPU code has no ConvTranspose2d and refuses 16-bit "
                                                  "concat: the port stands in")
        row["speedup_vs_cpu"] = row["samples_per_s"] / row["cpu_baseline"]["value"]
    eng.close()
    return row


def decode_line(steps=256, prompt=512, max_len=1024):
    """Greedy KV-cache decode (mh_decoder_*) on the headline architecture with
    textbook-key attention (the decode has no MuNet counterpart): prefill a
    [4, prompt] batch, then `steps` one-token steps back to back on the
    device (positions prompt .. prompt + steps - 1).  HBM roofline: per step
    every Linear weight row is streamed once (the embedding tables are only
    gathered) and every head reads its cached keys and values."""
    from munet_amd import models, synth
    from munet_amd.engine import Decoder, Engine
    cfg = models.decoder_config(**CFG, attention="textbook")
    params = models.init_params(cfg, "gpt", scope="bench_decode")
    ids = models.make_input(cfg, (B, prompt), "gpt", scope="bench_decode_in")
    eng = Engine(0).load(cfg, params).compile((B, prompt))
    del params
    dcd = Decoder(eng, B, max_len)
    dcd.prefill(ids, logits=False)
    dcd.generate(8)  # warm-up
    dcd.prefill(ids, logits=False)
    toks, ms = dcd.generate(steps)
    st = dcd.stats()
    d, L, H, V, C = cfg["d_model"], cfg["num_layers"], cfg["num_heads"], cfg["vocab"], cfg["ctx"]
    es = 2
    streamed = st["weight_bytes"] - (V + C) * d * es  # every weight row but the gathered tables
    avg_len = prompt + (steps + 1) / 2.0
    kv = 2.0 * L * B * d * es * avg_len  # K and V of every cached position, every layer
    per_step = streamed + kv
    t = ms * 1e-3 / steps
    row = dict(workload="gpt_decoder_decode (BASELINE configs[4] architecture, textbook-key attention)",
               batch=B, prompt=prompt, steps=steps, positions=[prompt, prompt + steps - 1], dtype="bf16",
               ms_per_step=t * 1e3, tokens_per_s=B / t, prefill_ms=st["last_prefill_ms"],
               kernels_per_step=st["kernels_per_step"],
               roofline=dict(bound="hbm", bytes_per_step=per_step, achieved=per_step / t / 1e9, peak=PEAK_HBM / 1e9,
                             unit="GB/s", frac=per_step / t / PEAK_HBM),
               tokens_sample=toks[:4, 0].tolist())
    dcd.close()
    eng.close()
    return row


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip BASELINE configs 0-3")
    ap.add_argument("--probe", default=None, help="run one kernel of the forward for rocprofv3 --pmc and exit "
                    "(with --config: an op name of that config's plan)")
    ap.add_argument("--config", default=None,
                    help="measure only this BASELINE config (mlp, cnn, encoder_bf16, encoder_fp16, unet, decode), "
                         "print its JSON row and exit (for profiling one config)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the single-GPU design and how the path would shard are in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import ctypes

    import torch

    from munet_amd import _lib, models
    from munet_amd.backend import HipBackend
    from munet_amd.engine import Engine

    if args.config:
        keys = {k: (i, c) for k, i, c in CONFIG_ROWS}
        if args.probe and args.config in keys:
            probe_config(torch, args.config, args.probe)
            return
        if args.config == "decode":
            row = decode_line()
        elif args.config in keys:
            idx, cpu_batch = keys[args.config]
            row = config_line(torch, args.config, idx, cpu_batch, args.steps, args.warmup, not args.no_cpu_baseline)
        else:
            sys.exit(f"bench: unknown config {args.config!r} (one of {sorted(keys) + ['decode']})")
        print(json.dumps({"config": args.config, **row}), flush=True)
        return

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

    s = timed_launches(eng, torch, args.steps, args.warmup)
    ms = s * 1e3
    tokens_s = B * T / s
    log(f"bench: {ms:.3f} ms/forward, {tokens_s:,.0f} tokens/s")
    # the timed forwards reran the resident input: no device error (token id
    # out of range) and the same logits as the first forward, bit for bit
    _lib.call("mh_check_device_errors")
    again = np.empty_like(logits)
    _lib.call("mh_copy", ctypes.c_void_p(eng.output_ptr()), again.ctypes.data_as(ctypes.c_void_p),
              ctypes.c_size_t(again.nbytes), 1, 0, ctypes.c_void_p(eng.stream()))
    if not np.array_equal(again.view(np.uint16), logits.view(np.uint16)):
        raise SystemExit("bench: repeated forwards changed the logits")

    # measured peaks beside the datasheet ones: the MFMA loop of peak.hip, a
    # read-only stream over 2 GiB, and a 1 GiB device-to-device copy
    hb = HipBackend(0)
    peak_mfma = hb.measure_mfma_peak(2, 16000)
    buf = torch.empty(1 << 30, device="cuda", dtype=torch.float16)
    buf.fill_(1.0)
    peak_read = hb.measure_hbm_read(buf, 5)
    src = buf[: 1 << 29]
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    peak_copy = 5 * 2.0 * src.numel() * 2 / (e0.elapsed_time(e1) * 1e-3)
    del src, dst, buf

    # per-op cost inside the forward (prefix-graph differences) picks the
    # dominant kernel; its launch duration is the mean over 20 back-to-back
    # launches of the forward's own op replayed from one graph between HIP
    # events on the engine stream (the dispatches a kernel trace of this
    # command shows)
    fwd_rows = categorise(eng.forward_op_times(20))
    for r in fwd_rows.values():
        r["per_fwd"] = r["t"] * r["count"]
    iso = categorise(eng.op_times(20))
    dom_f = max(fwd_rows.values(), key=lambda r: r["per_fwd"])
    dom = iso[dom_f["name"]]
    t_dom = dom["t"]
    if dom["flops"]:
        ach = dom["flops"] / t_dom
        roof = dict(bound="mfma", achieved=ach / 1e12, peak=PEAK_BF16 / 1e12, unit="TFLOP/s", frac=ach / PEAK_BF16,
                    peak_measured=peak_mfma / 1e12, frac_of_measured=ach / peak_mfma)
    else:
        ach = dom["bytes"] / t_dom
        roof = dict(bound="hbm", achieved=ach / 1e9, peak=PEAK_HBM / 1e9, unit="GB/s", frac=ach / PEAK_HBM,
                    peak_measured=peak_read / 1e9, frac_of_measured=ach / peak_read)
    roof.update(kernel=dom["name"], avg_us=t_dom * 1e6, launches_per_forward=dom["count"],
                work_per_launch=dom["flops"] or dom["bytes"],
                timing="20 back-to-back launches of the forward's own op from one graph between HIP events",
                in_forward_us_per_forward=dom_f["per_fwd"] * 1e6, share_of_forward=dom_f["per_fwd"] / s,
                traffic=measured_traffic(dom["name"]))

    kernels = {n: dict(avg_us=round(r["t"] * 1e6, 2), per_forward=r["count"],
                       tflops=round(r["flops"] / r["t"] / 1e12, 1) if r["flops"] else None,
                       gbs=round(r["bytes"] / r["t"] / 1e9, 1) if r["bytes"] else None) for n, r in iso.items()}
    # memory-bound ops carry their GB/s and HBM fraction both inside the
    # forward (prefix-graph differences) and alone
    for n, r in kernels.items():
        if r["gbs"]:
            r["hbm_frac"] = round(r["gbs"] * 1e9 / PEAK_HBM, 3)
    in_fwd = {n: dict(avg_us=round(r["t"] * 1e6, 2), per_forward=r["count"], us_per_forward=round(r["per_fwd"] * 1e6, 1),
                      tflops=round(r["flops"] / r["t"] / 1e12, 1) if r["flops"] and r["t"] > 0 else None,
                      gbs=round(r["bytes"] / r["t"] / 1e9, 1) if r["bytes"] and r["t"] > 0 else None,
                      hbm_frac=round(r["bytes"] / r["t"] / PEAK_HBM, 3) if r["bytes"] and r["t"] > 0 else None)
              for n, r in fwd_rows.items()}
    # the first op's prefix difference is the one-op graph's whole replay
    # time, graph launch overhead included
    first = op_category(eng.plan()["ops"][0])
    if first in in_fwd:
        in_fwd[first]["note"] = "first op of the forward: includes the graph launch overhead"
    gemm_f = [r for r in fwd_rows.values() if r["flops"] and r["name"] != "attention_causal"]
    gemm_frac_fwd = sum(r["flops"] * r["count"] for r in gemm_f) / sum(r["per_fwd"] for r in gemm_f) / PEAK_BF16
    gemm_i = [r for r in iso.values() if r["flops"] and r["name"] != "attention_causal"]
    gemm_frac_iso = sum(r["flops"] * r["count"] for r in gemm_i) / sum(r["t"] * r["count"] for r in gemm_i) / PEAK_BF16
    ln = iso["layer_norm"]

    cpu = None
    if not args.no_cpu_baseline:
        log("bench: timing the CPU baseline sample (MuNet's compiled code, then the port)")
        port = cpu_baseline_gpt()
        port["reference_check"] = reference_check()
        cpu = cpu_reference_gpt()
        if cpu is None:
            cpu = port
        else:
            cpu["port"] = port
        cpu["speedup_vs_cpu"] = tokens_s / cpu["value"]
    configs = None
    if not args.no_configs:
        configs = {}
        for key, idx, cpu_batch in CONFIG_ROWS:
            log(f"bench: config {key}")
            configs[key] = config_line(torch, key, idx, cpu_batch, args.steps, args.warmup, not args.no_cpu_baseline)
        log("bench: KV-cache decode")
        configs["decode"] = decode_line()
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
        "gemm_mfma_frac": gemm_frac_fwd,
        "gemm_mfma_frac_isolated": gemm_frac_iso,
        "layernorm_hbm_frac": (ln["bytes"] / ln["t"]) / PEAK_HBM,
        "layernorm_hbm_frac_in_forward": (ln["bytes"] / fwd_rows["layer_norm"]["t"]) / PEAK_HBM
        if fwd_rows["layer_norm"]["t"] > 0 else None,
        "layernorm_frac_of_measured_read": (ln["bytes"] / ln["t"]) / peak_read,
        "measured_peaks": {"mfma_bf16_tflops": peak_mfma / 1e12, "hbm_read_gbs": peak_read / 1e9,
                           "hbm_copy_gbs": peak_copy / 1e9},
        "kernels_in_forward": in_fwd,
        "kernels_isolated": kernels,
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
