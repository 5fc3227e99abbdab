"""LayerNorm folded across the GEMM boundary (bf16 engine): the embedding and
residual GEMM epilogues write row partials (mean, M2 per 16 columns) and the
next Linear normalises in its epilogue, LN(x) W = rstd (x (gamma (.) W) -
mean colsum(gamma (.) W)) + beta W.

The BASELINE initialisation (gamma = 1, beta = 0, zero biases) leaves most of
that algebra untouched, so these cases draw gamma ~ U(0.5, 1.5), beta and
every bias ~ N(0, 0.1), scale the token table to unit spread and shift the
position table by a constant, so that every row's mean is several spreads
from zero (the mean * colsum term then cancels most of the raw product).
The residual stream must stay resolvable in bf16 for any implementation to
match the reference: at mean 4 and spread 0.03 one bf16 ulp (0.031) is a
whole spread, and the unfolded engine misses the tolerance as much as the
folded one (measured 4.5e-2 and 4.9e-2); at spread 1 both stay near 1e-2.
Parity: the oracle (MuNet's unfolded, per-op rounded chain) within the bf16
tolerance, argmax where the reference gap is clear, and agreement with the
same engine run unfolded (MUNET_HIP_LN_FOLD=0).
"""
import numpy as np
import pytest

from munet_amd import models, synth
from munet_amd.engine import Engine
from oracle import models as omodels
from util import RTOL, assert_close, dec

pytestmark = pytest.mark.gpu


def _perturbed(cfg, scope, shift=0.0):
    params = models.init_params(cfg, "gpt" if cfg["type"] == "DecoderLM" else "xavier", scope=scope)
    rng = np.random.default_rng(11)
    dt = synth.BF16
    for name, shape, role, _info in models.param_specs(cfg):
        if role == "ln_w":
            params[name] = synth.encode(rng.uniform(0.5, 1.5, shape), dt)
        elif role in ("ln_b", "bias"):
            params[name] = synth.encode(rng.standard_normal(shape) * 0.1, dt)
        elif name.endswith("token_embed.weight"):
            params[name] = synth.encode(synth.decode(params[name], dt).astype(np.float64) * 50.0, dt)
        elif name.endswith("pos_embed.weight") and shift:
            params[name] = synth.encode(synth.decode(params[name], dt).astype(np.float64) + shift, dt)
    return params


def _argmax_check(y, y_ref, dt):
    a, b = dec(y, dt), dec(y_ref, dt)
    a2, b2 = a.reshape(-1, a.shape[-1]), b.reshape(-1, b.shape[-1])
    srt = np.sort(b2, axis=1)
    clear = (srt[:, -1] - srt[:, -2]) > RTOL[dt] * np.max(np.abs(b2))
    assert clear.sum() > 0
    assert np.array_equal(np.argmax(a2[clear], 1), np.argmax(b2[clear], 1))


@pytest.mark.parametrize("shift", [0.0, 4.0])
def test_decoder_folded_layer_norm_vs_oracle(orc, monkeypatch, shift):
    cfg = models.decoder_config(vocab=1000, ctx=128, d_model=256, num_heads=4, num_layers=2, ffn=1024)
    params = _perturbed(cfg, "lnfold", shift)
    ids = models.make_input(cfg, (2, 128), "gpt", scope="lnfold_in")
    eng = Engine(0).load(cfg, params).compile((2, 128))
    assert eng.stats()["ln_folds"] == 2 * 2 + 1  # ln_f too: the head (1000) is at most 4 d wide
    y = eng.run(ids)
    ref = omodels.forward(orc, cfg, params, ids)
    assert_close(y, ref, synth.BF16, what=f"folded decoder logits (shift {shift})")
    _argmax_check(y, ref, synth.BF16)
    # the same engine without the fold (LayerNorm kernels) agrees as closely
    monkeypatch.setenv("MUNET_HIP_LN_FOLD", "0")
    eng0 = Engine(0).load(cfg, params).compile((2, 128))
    assert eng0.stats()["ln_folds"] == 0
    y0 = eng0.run(ids)
    assert_close(y0, ref, synth.BF16, what="unfolded decoder logits")
    assert_close(y, y0, synth.BF16, what="folded vs unfolded")
    assert np.array_equal(y, eng.run(ids))  # deterministic replays


def test_encoder_block_folded_layer_norm_vs_oracle(orc):
    """A single pre-LN block: its input is the engine input (no producer to
    write partials), so ln1 stays a kernel and only ln2 folds."""
    cfg = models.block_config(d_model=256, num_heads=4, ffn=1024)
    params = _perturbed(cfg, "lnfold_blk")
    x = models.make_input(cfg, (4, 64, 256), "xavier", scope="lnfold_blk_in")
    eng = Engine(0).load(cfg, params).compile((4, 64, 256))
    assert eng.stats()["ln_folds"] == 1
    y = eng.run(x)
    ref = omodels.forward(orc, cfg, params, x)
    assert_close(y, ref, synth.BF16, what="encoder block (ln2 folded)")


@pytest.mark.parametrize("tile", ["216", "217", "208", "200", "202", "219"])
def test_folded_decoder_bit_identical_across_tiles(monkeypatch, tile):
    """Every pipelined tile accumulates in the same K order and combines a
    row's LayerNorm partials in the same order (four chunks, then pairwise,
    whether a row has 2 or 4 threads), so the folded decoder
    (LayerNorm-consumer, statistics-producer and head-split programs) gives
    the same bits on any forced tile as on the automatic choice: 216
    (256x192) and 217 (128x96, blocks split unevenly over eight waves) are
    the eight-wave tiles, 202 (64x64) and 217 have 4 threads per row."""
    cfg = models.decoder_config(vocab=1000, ctx=128, d_model=384, num_heads=6, num_layers=2, ffn=1536)
    params = _perturbed(cfg, "lnfold_tiles")
    ids = models.make_input(cfg, (2, 128), "gpt", scope="lnfold_tiles_in")
    y = Engine(0).load(cfg, params).compile((2, 128)).run(ids)
    monkeypatch.setenv("MUNET_HIP_GEMM_TILE", tile)
    e = Engine(0).load(cfg, params).compile((2, 128))
    assert e.stats()["ln_folds"] == 2 * 2 + 1
    assert np.array_equal(e.run(ids), y)


@pytest.mark.parametrize("head", ["linear", "linear_relu", "linear_nobias", "linear_k36"])
def test_linear_then_block_vs_oracle(orc, head):
    """bf16 Sequential[Linear, TransformerBlock]: a producer whose epilogue
    cannot write row partials (no residual, an activation, no bias, K % 8 != 0)
    leaves ln1 a kernel; the model compiles and matches the oracle."""
    in_f = 36 if head == "linear_k36" else 40
    lin = {"type": "Linear", "in_features": in_f, "out_features": 128, "bias": head != "linear_nobias"}
    layers = [lin] + ([{"type": "ReLU"}] if head == "linear_relu" else [])
    layers.append({"type": "TransformerBlock", "d_model": 128, "num_heads": 2, "ffn": 256, "causal": False})
    cfg = {"type": "Sequential", "dtype": "bfloat16", "layers": layers}
    params = models.init_params(cfg, "xavier", scope="lin_blk_" + head)
    x = synth.make_tensor("lin_blk_in", "x", (2, 32, in_f), synth.BF16, "normal")
    eng = Engine(0).load(cfg, params).compile((2, 32, in_f))
    assert eng.stats()["ln_folds"] == 1  # ln2 only
    y = eng.run(x)
    ref = omodels.forward(orc, cfg, params, x)
    assert_close(y, ref, synth.BF16, what=f"Linear -> TransformerBlock ({head})")


@pytest.mark.parametrize("d,heads", [(768, 12), (1008, 12)])
def test_decoder_fold_partial_counts_vs_oracle(orc, d, heads):
    """The consumer combines 16 partials per row at d = 768 (48-column
    groups) and 63 at d = 1008 (16-column groups, an odd count loaded two
    at a time with a clamped last pair)."""
    cfg = models.decoder_config(vocab=512, ctx=64, d_model=d, num_heads=heads, num_layers=2, ffn=2 * d)
    params = _perturbed(cfg, f"lnfold_parts_{d}")
    ids = models.make_input(cfg, (2, 64), "gpt", scope=f"lnfold_parts_in_{d}")
    eng = Engine(0).load(cfg, params).compile((2, 64))
    assert eng.stats()["ln_folds"] == 2 * 2 + 1
    y = eng.run(ids)
    ref = omodels.forward(orc, cfg, params, ids)
    assert_close(y, ref, synth.BF16, what=f"folded decoder d={d}")
    _argmax_check(y, ref, synth.BF16)
