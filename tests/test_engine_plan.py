"""Compile-time passes of the engine on a plan-only engine (no GPU):
fusion decisions, liveness-planned arena, zero-copy concat."""
import json

import numpy as np
import pytest

from munet_amd import _lib, models, synth
from munet_amd.engine import Engine


def _zero_params(cfg):
    dt = synth.DTYPE_CODES[cfg.get("dtype", "float32")]
    return {n: np.zeros(s, dtype=synth.storage_dtype(dt)) for n, s, _r, _i in models.param_specs(cfg)}


def _plan(cfg, in_shape):
    e = Engine(device=-1).load(cfg, _zero_params(cfg)).compile(in_shape)
    return e, e.plan()


def _check_arena(plan):
    vals = plan["values"]
    roots = [v for v in vals if v["alias_of"] < 0 and v["offset"] >= 0]
    for i, a in enumerate(roots):
        for b in roots[i + 1:]:
            live = not (a["last"] < b["def"] or b["last"] < a["def"])
            if live:
                sep = a["offset"] + a["bytes"] <= b["offset"] or b["offset"] + b["bytes"] <= a["offset"]
                assert sep, f"live values overlap in the arena: {a} {b}"
    assert plan["arena_bytes"] >= max(v["offset"] + v["bytes"] for v in roots)
    return sum(v["bytes"] for v in roots)


def test_mlp_plan_fuses_relu():
    cfg = models.mlp_config()
    e, p = _plan(cfg, (64, 784))
    kinds = [o["kind"] for o in p["ops"]]
    assert kinds == ["gemm", "gemm", "gemm"]
    assert [o["act"] for o in p["ops"]] == [1, 1, 0]
    _check_arena(p)
    assert e.out_shape == (64, 10)


def test_decoder_plan_structure_and_reuse():
    """bf16 decoder: both LayerNorms of every block fold into the Linear
    after them (the final one stays a kernel before the much wider vocabulary
    head); the embedding (whole-row statistics, [M, 1, 2]) and the residual
    GEMMs (per 32 columns at d = 128, [M, 4, 2]) write the f32 row partials
    that the folded Linear reads."""
    cfg = models.decoder_config(vocab=1000, ctx=256, d_model=128, num_heads=2, num_layers=3, ffn=512)
    assert cfg["dtype"] == "bfloat16"
    e, p = _plan(cfg, (2, 256))
    ops = p["ops"]
    kinds = [o["kind"] for o in ops]
    per_layer = ["qkv_gemm", "attention", "gemm", "gemm", "gemm"]
    assert kinds == ["embedding_pos"] + per_layer * 3 + ["layer_norm", "gemm"]
    st = e.stats()
    assert st["fused_epilogues"] == 3 * 3  # out_proj+resid, ffn0+gelu, ffn2+resid per layer
    assert st["ln_folds"] == 2 * 3
    assert not st["stream_out"]  # 2 MB of logits stay cacheable
    # producers: embedding, then out_proj and ffn.2 of every layer; consumers:
    # qkv, ffn.0 of every layer and the head; each stats value links one pair
    producers = [i for i, o in enumerate(ops) if o["stats_out"] >= 0]
    consumers = [i for i, o in enumerate(ops) if o["ln_stats"] >= 0]
    assert producers == [0] + [1 + 5 * l + j for l in range(3) for j in (2, 4)][:-1]
    assert consumers == [1 + 5 * l + j for l in range(3) for j in (0, 3)]
    for pi, ci in zip(producers, consumers):
        sv = ops[pi]["stats_out"]
        assert ops[ci]["ln_stats"] == sv and sv in ops[pi]["out"] and sv in ops[ci]["in"]
        assert p["values"][sv]["shape"] == [2 * 256, 1 if pi == 0 else 128 // 32, 2]
        assert p["values"][sv]["dtype"] == 0
    total = _check_arena(p)
    assert p["arena_bytes"] < total / 2  # liveness reuse
    assert e.out_shape == (2, 256, 1000)


def test_decoder_plan_without_ln_fold(monkeypatch):
    """MUNET_HIP_LN_FOLD=0 keeps the LayerNorm ops (the unfolded reference
    structure)."""
    monkeypatch.setenv("MUNET_HIP_LN_FOLD", "0")
    cfg = models.decoder_config(vocab=1000, ctx=256, d_model=128, num_heads=2, num_layers=3, ffn=512)
    e, p = _plan(cfg, (2, 256))
    kinds = [o["kind"] for o in p["ops"]]
    per_layer = ["layer_norm", "qkv_gemm", "attention", "gemm", "layer_norm", "gemm", "gemm"]
    assert kinds == ["embedding_pos"] + per_layer * 3 + ["layer_norm", "gemm"]
    assert e.stats()["ln_folds"] == 0
    assert all(o["stats_out"] < 0 and o["ln_stats"] < 0 for o in p["ops"])


def test_fp16_decoder_keeps_layer_norm():
    """The fold exists only on the bf16 fast epilogue."""
    cfg = models.decoder_config(vocab=1000, ctx=256, d_model=128, num_heads=2, num_layers=1, ffn=512,
                                dtype="float16")
    e, p = _plan(cfg, (2, 256))
    assert [o["kind"] for o in p["ops"]].count("layer_norm") == 3
    assert e.stats()["ln_folds"] == 0


@pytest.mark.parametrize("which", ["mlp", "decoder", "unet"])
def test_input_buffer_is_never_reused(which):
    """The input stays valid across repeated launches on a device-resident
    input: no other value may share its arena bytes, at any time."""
    if which == "mlp":
        cfg, shape = models.mlp_config(), (64, 784)
    elif which == "decoder":
        cfg, shape = models.decoder_config(vocab=1000, ctx=256, d_model=128, num_heads=2, num_layers=2, ffn=512), (2, 256)
    else:
        cfg, shape = models.unet_config(channels=(8, 16, 32), out_channels=2), (2, 3, 32, 32)
    _e, p = _plan(cfg, shape)
    vals = p["values"]
    inp = vals[p["input"]]
    lo, hi = inp["offset"], inp["offset"] + inp["bytes"]
    for i, v in enumerate(vals):
        if i == p["input"] or v["alias_of"] == p["input"] or v["offset"] < 0:
            continue
        assert v["offset"] + v["bytes"] <= lo or hi <= v["offset"], f"value {i} reuses the input's bytes: {v}"


def test_unet_zero_copy_concat():
    cfg = models.unet_config(channels=(8, 16, 32), out_channels=2)
    e, p = _plan(cfg, (2, 3, 32, 32))
    assert e.stats()["zero_copy_concats"] == 2
    assert not any(o["kind"] == "concat" for o in p["ops"])
    assert [o["kind"] for o in p["ops"]].count("conv_transpose2d") == 2
    _check_arena(p)
    assert e.out_shape == (2, 2, 32, 32)


def test_unet_plan_reads_the_image_and_writes_the_output_in_place():
    """A 16-bit UNet: the first convolution reads the NCHW image itself and
    the 1x1 head writes the NCHW output itself, so no layout conversion runs."""
    cfg = models.unet_config(channels=(64, 128, 256, 512), out_channels=2)
    e, p = _plan(cfg, (2, 3, 64, 64))
    kinds = [o["kind"] for o in p["ops"]]
    assert "nchw_to_nhwc" not in kinds and "nhwc_to_nchw" not in kinds
    assert kinds[0] == "conv2d" and kinds[-1] == "conv2d"
    assert p["values"][p["output"]]["layout"] == 0  # row-major NCHW
    _check_arena(p)
    assert e.out_shape == (2, 2, 64, 64)


def test_cnn_plan_layouts():
    """The CNN runs NHWC end to end with no layout copies: the first
    convolution reads the NCHW image in place, and the Flatten feeding the
    first Linear is that Linear reading the NHWC activation with permuted
    weight rows."""
    cfg = models.cnn_config()
    e, p = _plan(cfg, (32, 3, 32, 32))
    kinds = [o["kind"] for o in p["ops"]]
    assert "nchw_to_nhwc" not in kinds and "nhwc_to_nchw" not in kinds
    assert kinds.count("conv2d") == 2 and kinds.count("max_pool2d") == 2
    _check_arena(p)
    assert e.out_shape == (32, 10)


def test_full_gpt_plan_fits_and_reuses():
    """BASELINE config 5 shape contract: the plan for the 12-layer decoder."""
    cfg = models.decoder_config()
    e, p = _plan(cfg, (4, 1024))
    st = e.stats()
    assert st["ops"] == 1 + 12 * 5 + 2  # embedding, 5 per layer (both LayerNorms folded), ln_f, head
    assert st["ln_folds"] == 24
    assert st["stream_out"]  # 262 MB of logits: the head stores them non-temporally
    assert e.out_shape == (4, 1024, 32000)
    _check_arena(p)
    # logits (262 MB) + a few activations; far below one buffer per op
    assert st["arena_bytes"] < 400 * 2 ** 20


def test_engine_errors():
    cfg = models.mlp_config()
    params = _zero_params(cfg)
    del params["0.weight"]
    with pytest.raises(_lib.HipError, match="missing parameter '0.weight'"):
        Engine(device=-1).load(cfg, params).compile((64, 784))
    with pytest.raises(_lib.HipError, match="does not end in 784"):
        Engine(device=-1).load(cfg, _zero_params(cfg)).compile((64, 783))
    with pytest.raises(_lib.HipError, match="unsupported module type"):
        bad = {"type": "Sequential", "dtype": "float32", "layers": [{"type": "LSTM"}]}
        Engine(device=-1).load(bad, {}).compile((2, 3))


def test_fold_only_from_a_residual_producer():
    """A LayerNorm folds into its consumer only when its input comes from the
    embedding or a bias + residual GEMM with no activation (the only producer
    epilogue that writes row partials).  A plain Linear, a Linear + ReLU or a
    bias-free Linear before a bf16 TransformerBlock keeps ln1 as a kernel
    (ln2's producer, the out-projection with its residual, still folds)."""
    blk = {"type": "TransformerBlock", "d_model": 64, "num_heads": 2, "ffn": 128, "causal": False}
    for head in ([{"type": "Linear", "in_features": 40, "out_features": 64}],
                 [{"type": "Linear", "in_features": 40, "out_features": 64}, {"type": "ReLU"}],
                 [{"type": "Linear", "in_features": 40, "out_features": 64, "bias": False}],
                 [{"type": "Linear", "in_features": 36, "out_features": 64}]):
        cfg = {"type": "Sequential", "dtype": "bfloat16", "layers": head + [blk]}
        cfg["layers"][-1] = dict(blk)
        in_f = head[0]["in_features"]
        e, p = _plan(cfg, (2, 8, in_f))
        kinds = [o["kind"] for o in p["ops"]]
        assert kinds[1] == "layer_norm", kinds
        assert e.stats()["ln_folds"] == 1


def _params_for(cfg):
    return _zero_params(cfg)


@pytest.mark.parametrize("name,count", [
    ("blocks.0.attn.q_proj.bias", 127), ("blocks.0.ln1.bias", 100), ("blocks.0.ff.0.bias", 511),
    ("token_embed.weight", 999 * 128), ("pos_embed.weight", 255 * 128), ("head.bias", 999),
    ("ln_f.weight", 129)])
def test_wrong_sized_parameter_is_rejected(name, count):
    """Every parameter the engine uploads is checked against the element
    count its layer needs (the reference's loader checks every shape:
    src/inference_serialization.cpp:863-881)."""
    cfg = models.decoder_config(vocab=1000, ctx=256, d_model=128, num_heads=2, num_layers=1, ffn=512)
    p = _params_for(cfg)
    p[name] = np.zeros(count, dtype=np.uint16)
    with pytest.raises(_lib.HipError, match=f"parameter '{name}' has {count} elements"):
        Engine(device=-1).load(cfg, p).compile((2, 16))


def test_unknown_or_wrong_dtype_parameter_is_rejected():
    cfg = models.mlp_config((20, 16, 4))
    p = _params_for(cfg)
    p["9.weight"] = np.zeros((3, 3), np.float32)
    with pytest.raises(_lib.HipError, match="unknown parameter '9.weight'"):
        Engine(device=-1).load(cfg, p).compile((5, 20))
    p = _params_for(cfg)
    p["0.bias"] = np.zeros(16, np.int32)
    with pytest.raises(_lib.HipError, match="0.bias"):
        Engine(device=-1).load(cfg, p).compile((5, 20))
