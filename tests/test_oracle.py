"""Pins the CPU restatement (oracle/munet_cpu_ref.cpp) before it is trusted:

* against the golden vectors written from MuNet's own CPU code
  (tests/golden/make_golden.py; bit-exact);
* against oracle/_ref (MuNet's CPU sources compiled here) on fresh seeded
  cases, when that library is present (bit-exact);
* against closed forms and invariants the mathematics fixes;
* with planted mistakes (textbook attention instead of the reference's K
  reinterpretation, RNE instead of round-half-away fp16, a transposed operand)
  that these checks must reject.
"""
import glob
import os

import numpy as np
import pytest

from munet_amd import synth
from oracle import CpuOracle, available

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))
DT = {"f32": synth.F32, "f16": synth.F16, "bf16": synth.BF16}


def _dt_of(name):
    return DT[name.split("_")[-1]] if name.split("_")[-1] in DT else DT[[t for t in DT if f"_{t}_" in name][0]]


def _run_case(o, name, z):
    dt = _dt_of(name)
    if name.startswith("matmul_"):
        return o.matmul(z["a"], z["b"], dt)
    if name.startswith("linear3d_"):
        return o.linear(z["x"], z["w"], z["bias"], dt)
    if name.startswith("gelu_"):
        return o.gelu(z["x"], dt)
    if name.startswith("softmax_"):
        return o.softmax(z["x"], dt)
    if name.startswith("layer_norm_"):
        return o.layer_norm(z["x"], z["w"], z["b"], dt)
    if name.startswith("mha_"):
        p = {k.replace("_weight", ".weight").replace("_bias", ".bias"): z[k] for k in z.files if "proj" in k}
        return o.mha(z["x"], p, int(z["heads"]), bool(z["causal"]), dt)
    if name.startswith("conv2d_s2_"):
        return o.conv2d(z["x"], z["w"], z["b"], 2, 1, dt)
    if name.startswith("conv2d_"):
        return o.conv2d(z["x"], z["w"], z["b"], 1, 1, dt)
    if name.startswith("max_pool2d_"):
        return o.max_pool2d(z["x"], 2, 2, 0, dt)
    if name.startswith("upsample2d_"):
        return o.upsample2d(z["x"], 2, dt)
    if name.startswith("embedding_"):
        return o.embedding(z["ids"], z["w"], dt)
    if name.startswith("encode_"):
        return o.encode(z["x"], dt)
    raise KeyError(name)


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_restatement_matches_golden(orc, path):
    name = os.path.basename(path)[:-4]
    z = np.load(path)
    got = _run_case(orc, name, z)
    assert np.array_equal(got, z["out"]), f"{name}: restatement differs from MuNet's own output"


def test_golden_set_is_complete():
    names = {os.path.basename(p)[:-4].rsplit("_", 1)[0] for p in GOLDEN}
    for must in ("matmul", "linear3d", "gelu", "softmax", "layer_norm", "conv2d", "max_pool2d", "upsample2d",
                 "embedding", "encode"):
        assert must in names, must
    assert sum("mha_" in p for p in GOLDEN) == 12


@pytest.mark.skipif(not available("reference"), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("dt", [synth.F32, synth.F16, synth.BF16])
def test_restatement_matches_compiled_reference(orc, dt):
    ref = CpuOracle("reference")
    rng = np.random.default_rng(123 + dt)
    enc = lambda *s, sc=1.0: synth.encode(rng.standard_normal(s) * sc, dt)  # noqa: E731
    a, b = enc(41, 67), enc(67, 23)
    assert np.array_equal(orc.matmul(a, b, dt), ref.matmul(a, b, dt))
    a3, b3 = enc(3, 9, 17), enc(3, 17, 5)
    assert np.array_equal(orc.matmul(a3, b3, dt), ref.matmul(a3, b3, dt))
    x, bias = enc(19, 31), enc(31)
    for fn in ("relu", "sigmoid", "gelu", "softmax"):
        assert np.array_equal(getattr(orc, fn)(x, dt), getattr(ref, fn)(x, dt)), fn
    assert np.array_equal(orc.add(x, bias, dt), ref.add(x, bias, dt))
    assert np.array_equal(orc.layer_norm(x, bias, bias, dt), ref.layer_norm(x, bias, bias, dt))
    B, T, E, H = 2, 9, 12, 3
    xx = enc(B, T, E)
    p = {}
    for i, n in enumerate(("q_proj", "k_proj", "v_proj", "out_proj")):
        p[n + ".weight"], p[n + ".bias"] = enc(E, E, sc=0.4), enc(E, sc=0.1)
    for causal in (False, True):
        assert np.array_equal(orc.mha(xx, p, H, causal, dt), ref.mha(xx, p, H, causal, dt))
    cx, cw, cb = enc(2, 4, 7, 7), enc(5, 4, 3, 3, sc=0.3), enc(5)
    assert np.array_equal(orc.conv2d(cx, cw, cb, 1, 1, dt), ref.conv2d(cx, cw, cb, 1, 1, dt))


# ---- closed forms and invariants -------------------------------------------

def test_closed_forms(orc):
    for dt in (synth.F32, synth.F16, synth.BF16):
        ones = lambda *s: synth.encode(np.ones(s), dt)  # noqa: E731
        assert np.all(synth.decode(orc.matmul(ones(5, 24), ones(24, 3), dt), dt) == 24)
        assert np.all(synth.decode(orc.conv2d(ones(1, 2, 5, 5), ones(3, 2, 3, 3), None, 1, 0, dt), dt) == 18)
    g = orc.gelu(np.array([-2.0, 0.0, 2.0], np.float32), synth.F32)
    np.testing.assert_allclose(g, [-0.0643, 0.0, 1.9357], atol=5e-3)  # tests/test_nn.cpp:385-402
    x = synth.encode(np.random.default_rng(0).standard_normal((6, 300)) * 5 + 3, synth.F32)
    y = orc.layer_norm(x, np.ones(300, np.float32), np.zeros(300, np.float32), synth.F32)
    np.testing.assert_allclose(y.mean(1), 0, atol=1e-4)  # tests/test_nn.cpp:447-490
    np.testing.assert_allclose(y.var(1), 1, atol=2e-3)
    s = orc.softmax(x, synth.F32)
    np.testing.assert_allclose(s.sum(1), 1, atol=1e-6)


def test_codecs(orc):
    bits = np.arange(65536, dtype=np.uint16)
    # fp16 decode of every pattern == IEEE binary16 (numpy), NaN payloads aside
    d = orc.decode(bits, synth.F16)
    ref = bits.view(np.float16).astype(np.float32)
    ok = np.isnan(ref) | (d == ref)
    assert ok.all()
    assert np.array_equal(orc.decode(bits, synth.BF16).view(np.uint32), bits.astype(np.uint32) << 16)
    # fp16 encode rounds half away from zero (src/types.hpp:239-278)
    tie_up = np.float32(1 + 2 ** -11)            # exactly between 1 and 1+2^-10
    tie_even = np.float32(1 + 3 * 2 ** -11)      # between 1+2^-10 and 1+2^-9
    e = orc.encode(np.array([tie_up, -tie_up, tie_even], np.float32), synth.F16)
    assert list(e) == [0x3C01, 0xBC01, 0x3C02]
    # bf16 encode is round-to-nearest-even on the bits
    t = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32)
    assert list(orc.encode(t, synth.BF16)) == [0x3F80, 0x3F82]
    # the synthetic-data codecs write the same bits
    v = np.random.default_rng(1).standard_normal(10000).astype(np.float32) * 100
    for dt in (synth.F16, synth.BF16):
        assert np.array_equal(synth.encode(v, dt), orc.encode(v, dt))


# ---- planted mistakes the checks must catch -----------------------------------

def _golden(name):
    return np.load(os.path.join(HERE, "golden", name + ".npz"))


def test_textbook_attention_is_rejected():
    """Reading K as a proper [T, hd] per head (what a 'fixed' MHA would do)
    must not reproduce the reference's output."""
    z = _golden("mha_f32_c0_B2T5E8H2")
    x, H = z["x"].astype(np.float64), int(z["heads"])
    B, T, E = x.shape
    hd = E // H
    W = lambda n: z[n + "_weight"].astype(np.float64)  # noqa: E731
    Bv = lambda n: z[n + "_bias"].astype(np.float64)  # noqa: E731
    q, k, v = (x @ W(n) + Bv(n) for n in ("q_proj", "k_proj", "v_proj"))
    sp = lambda t: t.reshape(B, T, H, hd).transpose(0, 2, 1, 3)  # noqa: E731
    s = sp(q) @ sp(k).transpose(0, 1, 3, 2) / np.sqrt(hd)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ctx = (p @ sp(v)).transpose(0, 2, 1, 3).reshape(B, T, E)
    textbook = ctx @ W("out_proj") + Bv("out_proj")
    assert np.max(np.abs(textbook - z["out"])) > 1e-2


def test_rne_fp16_is_rejected(orc):
    z = _golden("encode_f16")
    rne = z["x"].astype(np.float16).view(np.uint16)
    assert not np.array_equal(rne, z["out"])
    assert np.array_equal(orc.encode(z["x"], synth.F16), z["out"])


def test_transposed_operand_is_rejected(orc):
    z = _golden("matmul_f32")
    a, b = z["a"], z["b"]
    wrong = orc.matmul(a, np.ascontiguousarray(b.reshape(b.shape[1], b.shape[0]).T), synth.F32)
    assert not np.array_equal(wrong, z["out"])
