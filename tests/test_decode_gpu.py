"""KV-cache decode (mh_decoder_*, decode.hip) and the textbook-key attention
it runs, against the CPU restatement's textbook mode (oracle mha_core with
textbook=True, pinned in test_oracle.py against torch's float64
scaled_dot_product_attention and by the causal prefix property; MuNet itself
has no per-position-key attention, so there is no MuNet vector for it).

Tolerances as the engine tests: normwise 2e-2 for bf16/fp16, 1e-4 fp32;
argmax equal wherever the reference's top-1/top-2 gap is clear.  At the
headline size (12 layers, d 768, V 32000, B 4, 1024 positions) the decode is
checked through properties: every step's logits equal the engine's own
prefill forward of the same tokens at that position (to the tolerance), and
generate() repeats step()'s greedy tokens exactly.
"""
import numpy as np
import pytest

from munet_amd import models, synth
from munet_amd.backend import empty, to_device, to_host
from munet_amd.engine import Decoder, Engine
from oracle import models as omodels
from util import RTOL, assert_close, dec, rand

pytestmark = pytest.mark.gpu

F32, F16, BF16 = synth.F32, synth.F16, synth.BF16


@pytest.mark.parametrize("dt", [BF16, F16, F32])
@pytest.mark.parametrize("B,T,H,hd", [(2, 64, 2, 64), (1, 77, 3, 64), (2, 130, 2, 64), (1, 1, 2, 64),
                                      (2, 40, 2, 32)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_textbook_core(hip, orc, dt, B, T, H, hd, causal):
    """Textbook keys: hd 64 16-bit runs the flash kernel's row-staged K
    variant (any T: ragged tiles are row-masked), the rest the generic
    kernel."""
    E = H * hd
    q2, k2, v2 = rand((B * T, E), dt, 60), rand((B * T, E), dt, 61), rand((B * T, E), dt, 62)
    ref = orc.mha_core(q2, k2, v2, B, T, H, causal, dt, textbook=True)
    # device layout: head-split [B, H, T, hd]
    split = lambda a: np.ascontiguousarray(a.reshape(B, T, H, hd).transpose(0, 2, 1, 3))
    q, k, v = (to_device(split(a), dt) for a in (q2, k2, v2))
    ctx = empty((B * T, E), dt)
    hip.attention_textbook(q, k, v, ctx, B, H, T, hd, causal)
    assert_close(to_host(ctx, dt), ref, dt, what="attention_textbook")


def _small(dt="bfloat16", layers=2):
    return models.decoder_config(vocab=500, ctx=96, d_model=128, num_heads=2, num_layers=layers, ffn=256, dtype=dt,
                                 attention="textbook")


def _argmax_clear(y, ref, dt):
    a = dec(y, dt).reshape(-1, y.shape[-1])
    b = dec(ref, dt).reshape(-1, ref.shape[-1])
    srt = np.sort(b, axis=1)
    clear = (srt[:, -1] - srt[:, -2]) > RTOL[dt] * np.max(np.abs(b))
    assert np.array_equal(np.argmax(a[clear], 1), np.argmax(b[clear], 1))
    return int(clear.sum())


@pytest.mark.parametrize("dt", ["bfloat16", "float16", "float32"])
def test_textbook_prefill_vs_oracle(orc, dt):
    """The engine's forward of a textbook DecoderLM (its prefill) against the
    restatement's textbook decoder."""
    cfg = _small(dt)
    d = synth.DTYPE_CODES[dt]
    p = models.init_params(cfg, "gpt", scope="tbp")
    ids = models.make_input(cfg, (2, 40), "gpt", scope="tbp_in")
    eng = Engine(0).load(cfg, p).compile(ids.shape)
    y = eng.run(ids)
    ref = omodels.forward(orc, cfg, p, ids)
    assert_close(y, ref, d, what="textbook prefill")
    _argmax_clear(y, ref, d)


def _steps_vs_oracle(orc, cfg, B, max_len, scope, T0=20, n=12):
    """Prefill T0 tokens, then n greedy steps; the oracle runs the whole fed
    sequence at once (teacher forcing on the decoder's own tokens) and each
    step's logits must match its position's row."""
    d = synth.DTYPE_CODES[cfg["dtype"]]
    p = models.init_params(cfg, "gpt", scope=scope)
    prompt = models.make_input(cfg, (B, T0), "gpt", scope=scope + "_in")
    eng = Engine(0).load(cfg, p).compile((B, T0))
    dcd = Decoder(eng, B, max_len)
    pre = dcd.prefill(prompt)
    assert dcd.position() == T0
    fed = [np.argmax(dec(pre[:, -1], d), axis=-1).astype(np.int32)]
    logits = []
    for i in range(n):
        lg, nxt = dcd.step()
        logits.append(lg)
        fed.append(nxt)
    assert dcd.position() == T0 + n
    seq = np.concatenate([prompt, np.stack(fed[:n], axis=1)], axis=1)
    ref = omodels.forward(orc, cfg, p, seq)
    assert_close(pre, ref[:, :T0], d, what="prefill logits")
    got = np.stack(logits, axis=1)  # [B, n, V]
    assert_close(got, ref[:, T0:], d, what="decode logits")
    _argmax_clear(got, ref[:, T0:], d)


@pytest.mark.parametrize("dt", ["bfloat16", "float16", "float32"])
def test_decode_steps_vs_oracle(orc, dt):
    _steps_vs_oracle(orc, _small(dt), 2, 64, "tbd")


@pytest.mark.parametrize("case", ["wide_batch_bf16", "long_cache_f32", "four_wave_f16", "four_wave_f32",
                                  "head_dim_32_bf16", "head_dim_48_f32_long_prompt"])
def test_decode_launch_shapes_vs_oracle(orc, case):
    """The step's other launch shapes against the oracle:
    wide_batch_bf16: batch 8 at d 512 (the 16-row kernels, and B*d > 3072,
    so the out-projection combines the attention shares in its input-stage
    loop instead of loading them ahead of the weights);
    long_cache_f32: a 1280-position cache with a 1100-token prompt (the
    steps run the five-block graph: five 256-key shares per head, the same
    combine loop);
    four_wave_f16 / four_wave_f32: FFN down with K past 128 chunks (its K
    split over the block's four waves), batches 5 and 3, and a vocabulary of
    8192 (the head's four-columns-per-row kernel);
    head_dim_32_bf16 / head_dim_48_f32_long_prompt: heads narrower than the
    attention kernel's eight lanes of 8 dimensions (lanes past the head
    dimension masked), the second with a 300-token prompt so that the keys
    span several waves and two 256-key blocks."""
    if case == "wide_batch_bf16":
        cfg = models.decoder_config(vocab=500, ctx=96, d_model=512, num_heads=8, num_layers=2, ffn=1024,
                                    dtype="bfloat16", attention="textbook")
        _steps_vs_oracle(orc, cfg, 8, 64, "dls_wb")
    elif case == "long_cache_f32":
        cfg = models.decoder_config(vocab=500, ctx=1280, d_model=128, num_heads=2, num_layers=2, ffn=256,
                                    dtype="float32", attention="textbook")
        _steps_vs_oracle(orc, cfg, 2, 1280, "dls_lc", T0=1100, n=6)
    elif case == "head_dim_32_bf16":
        cfg = models.decoder_config(vocab=500, ctx=96, d_model=128, num_heads=4, num_layers=2, ffn=256,
                                    dtype="bfloat16", attention="textbook")
        _steps_vs_oracle(orc, cfg, 2, 64, "dls_hd32")
    elif case == "head_dim_48_f32_long_prompt":
        cfg = models.decoder_config(vocab=500, ctx=320, d_model=96, num_heads=2, num_layers=2, ffn=192,
                                    dtype="float32", attention="textbook")
        _steps_vs_oracle(orc, cfg, 2, 320, "dls_hd48", T0=300, n=6)
    else:
        dt = "float16" if case.endswith("f16") else "float32"
        cfg = models.decoder_config(vocab=8192, ctx=96, d_model=128, num_heads=2, num_layers=2,
                                    ffn=1536 if dt == "float16" else 1024, dtype=dt, attention="textbook")
        _steps_vs_oracle(orc, cfg, 5 if dt == "float16" else 3, 64, "dls_" + case)


def test_decode_across_key_block_boundary(orc):
    """The step at position p runs the graph with p // 256 + 1 attention
    blocks (those holding keys 0..p), the out-projection combining that
    many shares: steps at positions 250..261 switch graphs at 256, against
    the oracle, and generate() across the switch repeats the single steps'
    tokens."""
    cfg = models.decoder_config(vocab=500, ctx=640, d_model=128, num_heads=2, num_layers=2, ffn=256,
                                dtype="bfloat16", attention="textbook")
    _steps_vs_oracle(orc, cfg, 2, 600, "dls_kb", T0=250, n=12)
    p = models.init_params(cfg, "gpt", scope="dls_kb")
    prompt = models.make_input(cfg, (2, 250), "gpt", scope="dls_kb_in")
    eng = Engine(0).load(cfg, p).compile((2, 250))
    dcd = Decoder(eng, 2, 600)
    assert dcd.stats()["step_graphs"] == 3
    dcd.prefill(prompt, logits=False)
    toks = [dcd.step()[1] for _ in range(12)]
    dcd.prefill(prompt, logits=False)
    gen, _ = dcd.generate(12)
    assert np.array_equal(gen, np.stack(toks))


def test_decode_explicit_ids_and_generate_repeat_step(orc):
    """step(ids) feeds the given tokens; generate(n) after the same prefill
    repeats step()'s greedy tokens bit for bit."""
    cfg = _small()
    p = models.init_params(cfg, "gpt", scope="tbg")
    B, T0, n = 3, 17, 9
    prompt = models.make_input(cfg, (B, T0), "gpt", scope="tbg_in")
    eng = Engine(0).load(cfg, p).compile((B, T0))
    dcd = Decoder(eng, B, 48)
    dcd.prefill(prompt, logits=False)
    toks = [dcd.step()[1] for _ in range(n)]
    dcd.prefill(prompt, logits=False)
    gen, ms = dcd.generate(n)
    assert ms > 0
    assert np.array_equal(gen, np.stack(toks))
    # explicit ids: the logits of feeding token t at position T0 equal the
    # oracle's row T0 for the sequence prompt + t
    dcd.prefill(prompt, logits=False)
    t = np.array([5, 77, 499], dtype=np.int32)
    lg, _ = dcd.step(t)
    ref = omodels.forward(orc, cfg, p, np.concatenate([prompt, t[:, None]], axis=1))
    assert_close(lg, ref[:, T0], synth.BF16, what="explicit-id step")
    st = dcd.stats()
    assert st["batch"] == B and st["position"] == T0 + 1 and st["prefill_instances"] == 1


def test_decode_mixed_calls_match_single_steps():
    """The greedy choices of one call are fed back by the next step's first
    kernel (or by the flush at the end of a call): prefill, generate(4),
    step(), step(explicit ids), generate(3), step() give the tokens and
    positions of the same sequence of single steps."""
    cfg = _small()
    p = models.init_params(cfg, "gpt", scope="tbm")
    B, T0 = 2, 11
    prompt = models.make_input(cfg, (B, T0), "gpt", scope="tbm_in")
    eng = Engine(0).load(cfg, p).compile((B, T0))
    dcd = Decoder(eng, B, 40)
    t = np.array([42, 7], dtype=np.int32)

    dcd.prefill(prompt, logits=False)
    ref = [dcd.step()[1] for _ in range(5)]
    ref.append(dcd.step(t)[1])
    ref += [dcd.step()[1] for _ in range(4)]
    assert dcd.position() == T0 + 10

    dcd.prefill(prompt, logits=False)
    got = list(dcd.generate(4)[0])
    got.append(dcd.step()[1])
    assert dcd.position() == T0 + 5
    got.append(dcd.step(t)[1])
    got += list(dcd.generate(3)[0])
    got.append(dcd.step()[1])
    assert dcd.position() == T0 + 10
    assert np.array_equal(np.stack(got), np.stack(ref))


def test_decoder_errors():
    cfg = _small()
    p = models.init_params(cfg, "gpt", scope="tbe")
    eng = Engine(0).load(cfg, p).compile((2, 8))
    with pytest.raises(Exception, match="max_len"):
        Decoder(eng, 2, 97)  # past ctx
    dcd = Decoder(eng, 2, 16)
    with pytest.raises(Exception, match="prefill first"):
        dcd.step()
    with pytest.raises(Exception, match="prompt length"):
        dcd.prefill(np.zeros((2, 17), np.int32))
    dcd.prefill(np.zeros((2, 15), np.int32), logits=False)
    dcd.step()
    with pytest.raises(Exception, match="past max_len"):
        dcd.step()
    with pytest.raises(Exception, match="out of range"):
        dcd.prefill(np.full((2, 4), 500, np.int32), logits=False)
    munet = models.decoder_config(vocab=500, ctx=96, d_model=128, num_heads=2, num_layers=1, ffn=256)
    e2 = Engine(0).load(munet, models.init_params(munet, "gpt", scope="tbe2")).compile((2, 8))
    with pytest.raises(Exception, match="textbook"):
        Decoder(e2, 2, 16)


def test_decode_full_config_vs_oracle(orc):
    """Headline architecture (12 layers, d 768, H 12, V 32000, B 4): a
    24-token prompt and 8 greedy steps against the restatement's textbook
    decoder on the fed sequence."""
    _steps_vs_oracle(orc, models.decoder_config(attention="textbook"), 4, 64, "tbfo", T0=24, n=8)


def test_decode_full_config_consistent_with_prefill():
    """Headline size (12 layers, d 768, H 12, V 32000, B 4): prefill 1000
    tokens, 24 greedy steps; the engine's own forward of the 1024 fed tokens
    gives the same logits at positions 1000..1023 (to the tolerance, argmax
    equal where clear), and generate() repeats the greedy tokens."""
    cfg = models.decoder_config(attention="textbook")
    p = models.init_params(cfg, "gpt", scope="tbf")
    B, T0, n = 4, 1000, 24
    prompt = models.make_input(cfg, (B, T0), "gpt", scope="tbf_in")
    eng = Engine(0).load(cfg, p).compile((B, 1024), expected_input_shape=(B, -1))
    dcd = Decoder(eng, B, 1024)
    pre = dcd.prefill(prompt)
    fed = [np.argmax(dec(pre[:, -1], BF16), axis=-1).astype(np.int32)]
    logits = []
    for _ in range(n):
        lg, nxt = dcd.step()
        logits.append(lg)
        fed.append(nxt)
    seq = np.concatenate([prompt, np.stack(fed[:n], axis=1)], axis=1)
    full = eng.run(seq)
    got = np.stack(logits, axis=1)
    assert np.all(np.isfinite(dec(got, BF16)))
    assert_close(got, full[:, T0:], BF16, what="decode vs prefill forward")
    assert _argmax_clear(got, full[:, T0:], BF16) > 0
    dcd.prefill(prompt, logits=False)
    gen, _ = dcd.generate(n)
    assert np.array_equal(gen, np.stack(fed[1:n + 1]))
