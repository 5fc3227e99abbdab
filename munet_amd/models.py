"""Module-tree configs, parameter specs and seeded initialisation for the five
BASELINE workloads.

Configs use the reference's serialized ``__config__`` schema
(src/inference_serialization.cpp:762-860: ``Sequential``/``Linear``/
``Conv2d``/``MaxPool2d``/``ReLU``/``GELU``/``Flatten``/``Embedding``/
``LayerNorm``/``MultiHeadAttention``/``Upsample``) plus three composite types
the reference only expresses as Python demo modules:

* ``TransformerBlock`` - pre-LN block ``x + attn(ln1(x))``, ``x + ff(ln2(x))``
  with ``ff = Sequential(Linear, GELU, Linear)``
  (demos/multigpu/gpt3_multi_gpu_demo.py:89-114,
  demos/transformers/decoder_block_demo.py:6-24).
* ``DecoderLM`` - token + position embedding gather, causal blocks, final
  LayerNorm, vocabulary head (gpt3_multi_gpu_demo.py:117-172; ids instead of
  one-hot so nn::Embedding takes its gather path, src/nn/linear.hpp:95).
* ``UNet`` / ``ConvTranspose2d`` - build-defined (the reference has no
  transposed convolution; see the UNet section of the design notes).

Parameter names follow ``Module::named_parameters`` (src/core/module.hpp:
95-107): ``<child>.<param>`` with Sequential children named by index.
"""
from __future__ import annotations

import copy
import math

import numpy as np

from . import synth


# ---- configs ---------------------------------------------------------------

def mlp_config(sizes=(784, 256, 256, 10), dtype="float32"):
    layers = []
    for i, (a, b) in enumerate(zip(sizes[:-1], sizes[1:])):
        layers.append({"type": "Linear", "in_features": a, "out_features": b, "bias": True})
        if i < len(sizes) - 2:
            layers.append({"type": "ReLU"})
    return {"type": "Sequential", "dtype": dtype, "layers": layers}


def cnn_config(dtype="float32", in_ch=3, hw=32, c1=32, c2=64, hidden=128, classes=10):
    flat = c2 * (hw // 4) * (hw // 4)
    return {"type": "Sequential", "dtype": dtype, "layers": [
        {"type": "Conv2d", "in_channels": in_ch, "out_channels": c1, "kernel_size": 3, "stride": 1, "padding": 1},
        {"type": "ReLU"},
        {"type": "MaxPool2d", "kernel_size": 2, "stride": 2, "padding": 0},
        {"type": "Conv2d", "in_channels": c1, "out_channels": c2, "kernel_size": 3, "stride": 1, "padding": 1},
        {"type": "ReLU"},
        {"type": "MaxPool2d", "kernel_size": 2, "stride": 2, "padding": 0},
        {"type": "Flatten"},
        {"type": "Linear", "in_features": flat, "out_features": hidden, "bias": True},
        {"type": "ReLU"},
        {"type": "Linear", "in_features": hidden, "out_features": classes, "bias": True},
    ]}


def block_config(d_model=512, num_heads=8, ffn=2048, causal=False, dtype="bfloat16", eps=1e-5):
    return {"type": "TransformerBlock", "dtype": dtype, "d_model": d_model,
            "num_heads": num_heads, "ffn": ffn, "causal": causal, "eps": eps}


def decoder_config(vocab=32000, ctx=1024, d_model=768, num_heads=12, num_layers=12,
                   ffn=3072, dtype="bfloat16", eps=1e-5, attention="munet"):
    """attention: "munet" (the reference's key reading) or "textbook"
    (per-position keys: the attention the KV-cache decoder runs)."""
    cfg = {"type": "DecoderLM", "dtype": dtype, "vocab": vocab, "ctx": ctx,
           "d_model": d_model, "num_heads": num_heads, "num_layers": num_layers,
           "ffn": ffn, "eps": eps}
    if attention != "munet":
        cfg["attention"] = attention
    return cfg


def unet_config(dtype="float16", in_channels=3, channels=(64, 128, 256, 512), out_channels=2):
    return {"type": "UNet", "dtype": dtype, "in_channels": in_channels,
            "channels": list(channels), "out_channels": out_channels}


# The five BASELINE.json workloads (configs[0..4]).
def baseline_workloads():
    return {
        "mlp": dict(config=mlp_config(), input_shape=(64, 784), init="mlp"),
        "cnn": dict(config=cnn_config(), input_shape=(32, 3, 32, 32), init="he"),
        "encoder_bf16": dict(config=block_config(dtype="bfloat16"), input_shape=(8, 256, 512), init="xavier"),
        "encoder_fp16": dict(config=block_config(dtype="float16"), input_shape=(8, 256, 512), init="xavier"),
        "unet": dict(config=unet_config(), input_shape=(8, 3, 128, 128), init="he"),
        "gpt": dict(config=decoder_config(), input_shape=(4, 1024), init="gpt"),
    }


# ---- parameter specs -------------------------------------------------------

def _linear(prefix, i, o, bias=True):
    specs = [(prefix + "weight", (i, o), "linear_w", {"fan_in": i, "fan_out": o})]
    if bias:
        specs.append((prefix + "bias", (o,), "bias", {}))
    return specs


def _conv(prefix, ic, oc, k):
    return [(prefix + "weight", (oc, ic, k, k), "conv_w", {"fan_in": ic * k * k, "fan_out": oc * k * k}),
            (prefix + "bias", (oc,), "bias", {})]


def _convt(prefix, ic, oc, k):
    return [(prefix + "weight", (ic, oc, k, k), "conv_w", {"fan_in": ic * k * k, "fan_out": oc * k * k}),
            (prefix + "bias", (oc,), "bias", {})]


def _ln(prefix, d):
    return [(prefix + "weight", (d,), "ln_w", {}), (prefix + "bias", (d,), "ln_b", {})]


def _mha(prefix, e):
    out = []
    for p in ("q_proj", "k_proj", "v_proj", "out_proj"):
        out += _linear(f"{prefix}{p}.", e, e)
    return out


def _block(prefix, cfg):
    d, f = cfg["d_model"], cfg["ffn"]
    return (_ln(prefix + "ln1.", d) + _mha(prefix + "attn.", d) + _ln(prefix + "ln2.", d)
            + _linear(prefix + "ff.0.", d, f) + _linear(prefix + "ff.2.", f, d))


def unet_layers(cfg):
    """Ordered (name, kind, ic, oc, k, stride, pad) of the build-defined UNet."""
    ch = cfg["channels"]
    L = len(ch)
    out = []
    prev = cfg["in_channels"]
    for l, c in enumerate(ch):
        out.append((f"enc{l}.0", "conv", prev, c, 3, 1, 1))
        out.append((f"enc{l}.1", "conv", c, c, 3, 1, 1))
        if l < L - 1:
            out.append((f"down{l}", "conv", c, c, 3, 2, 1))
        prev = c
    for l in range(L - 2, -1, -1):
        c = ch[l]
        out.append((f"up{l}", "convt", ch[l + 1], c, 2, 2, 0))
        out.append((f"dec{l}.0", "conv", 2 * c, c, 3, 1, 1))
        out.append((f"dec{l}.1", "conv", c, c, 3, 1, 1))
    out.append(("head", "conv", ch[0], cfg["out_channels"], 1, 1, 0))
    return out


def param_specs(cfg, prefix=""):
    t = cfg["type"]
    if t == "Sequential":
        out = []
        for i, layer in enumerate(cfg["layers"]):
            out += param_specs(layer, f"{prefix}{i}.")
        return out
    if t == "Linear":
        return _linear(prefix, cfg["in_features"], cfg["out_features"], cfg.get("bias", True))
    if t == "Conv2d":
        return _conv(prefix, cfg["in_channels"], cfg["out_channels"], cfg["kernel_size"])
    if t == "LayerNorm":
        return _ln(prefix, cfg["normalized_shape"])
    if t == "Embedding":
        return [(prefix + "weight", (cfg["num_embeddings"], cfg["embedding_dim"]), "embed", {})]
    if t == "MultiHeadAttention":
        return _mha(prefix, cfg["embed_dim"])
    if t == "TransformerBlock":
        return _block(prefix, cfg)
    if t == "DecoderLM":
        d = cfg["d_model"]
        out = [(prefix + "token_embed.weight", (cfg["vocab"], d), "embed", {}),
               (prefix + "pos_embed.weight", (cfg["ctx"], d), "embed", {})]
        for i in range(cfg["num_layers"]):
            out += _block(f"{prefix}blocks.{i}.", cfg)
        out += _ln(prefix + "ln_f.", d) + _linear(prefix + "head.", d, cfg["vocab"])
        return out
    if t == "UNet":
        out = []
        for name, kind, ic, oc, k, _s, _p in unet_layers(cfg):
            out += (_conv if kind == "conv" else _convt)(f"{prefix}{name}.", ic, oc, k)
        return out
    return []  # parameter-free layers


def init_params(cfg, scheme, scope="model", base_seed=synth.BASE_SEED):
    """Seeded weights in the config dtype (BASELINE.json init schemes)."""
    dt = synth.DTYPE_CODES[cfg.get("dtype", "float32")]
    params = {}
    for name, shape, role, info in param_specs(cfg):
        kw = {"base_seed": base_seed}
        if role in ("bias", "ln_b"):
            kind = "zeros"
        elif role == "ln_w":
            kind = "ones"
        elif scheme == "gpt":
            kind, kw["std"] = "normal", 0.02
        elif scheme == "mlp":
            kind, kw["std"] = "normal", math.sqrt(1.0 / info.get("fan_in", shape[-1]))
        elif scheme == "he":
            kind, kw["std"] = "normal", math.sqrt(2.0 / info.get("fan_in", shape[-1]))
        elif scheme == "xavier":
            fi, fo = info.get("fan_in", shape[0]), info.get("fan_out", shape[-1])
            lim = math.sqrt(6.0 / (fi + fo))
            kind, kw["low"], kw["high"] = "uniform", -lim, lim
        else:
            raise ValueError(scheme)
        params[name] = synth.make_tensor(scope, name, shape, dt, kind, **kw)
    return params


def make_input(cfg, shape, scheme, scope="input", base_seed=synth.BASE_SEED):
    dt = synth.DTYPE_CODES[cfg.get("dtype", "float32")]
    if cfg["type"] == "DecoderLM":
        return synth.make_tensor(scope, "ids", shape, synth.I32, "randint",
                                 high=cfg["vocab"], base_seed=base_seed)
    if scheme == "mlp":
        return synth.make_tensor(scope, "x", shape, dt, "uniform", base_seed=base_seed)
    return synth.make_tensor(scope, "x", shape, dt, "normal", base_seed=base_seed)


def output_shape(cfg, in_shape):
    t = cfg["type"]
    if t == "DecoderLM":
        return tuple(in_shape) + (cfg["vocab"],)
    if t == "TransformerBlock":
        return tuple(in_shape)
    if t == "UNet":
        return (in_shape[0], cfg["out_channels"], in_shape[2], in_shape[3])
    shape = list(in_shape)
    for layer in cfg["layers"]:
        lt = layer["type"]
        if lt == "Linear":
            shape[-1] = layer["out_features"]
        elif lt == "Conv2d":
            k, s, p = layer["kernel_size"], layer["stride"], layer["padding"]
            shape = [shape[0], layer["out_channels"], (shape[2] + 2 * p - k) // s + 1, (shape[3] + 2 * p - k) // s + 1]
        elif lt == "MaxPool2d":
            k, s, p = layer["kernel_size"], layer["stride"], layer["padding"]
            shape = [shape[0], shape[1], (shape[2] + 2 * p - k) // s + 1, (shape[3] + 2 * p - k) // s + 1]
        elif lt == "Flatten":
            shape = [shape[0], int(np.prod(shape[1:]))]
        elif lt == "Upsample":
            f = layer["scale_factor"]
            shape = [shape[0], shape[1], shape[2] * f, shape[3] * f]
    return tuple(shape)


def with_dtype(cfg, dtype):
    c = copy.deepcopy(cfg)
    c["dtype"] = dtype
    return c
