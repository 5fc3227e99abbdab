"""Op-level parity: every HIP entry point against the CPU restatement of
MuNet's CPU backend (oracle/munet_cpu_ref.cpp) on the same seeded inputs.

Tolerances: normwise rel 1e-4 for fp32, 2e-2 for
fp16/bf16; data movement, indexing and argmax bit-exact.
"""
import numpy as np
import pytest

from munet_amd import synth
from munet_amd.backend import BroadcastInfo, compute_broadcast, contiguous_strides, empty, to_device, to_host
from oracle import ADD, DIV, MUL, SUB
from util import assert_close, dec, rand

pytestmark = pytest.mark.gpu

F32, F16, BF16, I32 = synth.F32, synth.F16, synth.BF16, synth.I32
DTS = [F32, F16, BF16]


def _mm_operand(shape_mk, trans, dt, seed):
    m, k = shape_mk
    x = rand((m, k), dt, seed)
    return np.ascontiguousarray(x.T) if trans else x


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("M,K,N", [(64, 784, 256), (37, 53, 29), (128, 256, 10), (1, 8, 1), (300, 200, 130)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul(hip, orc, dt, M, K, N, ta, tb):
    a = rand((M, K), dt, 1)
    b = rand((K, N), dt, 2)
    a_st = np.ascontiguousarray(synth.decode(a, dt).T) if ta else synth.decode(a, dt)
    b_st = np.ascontiguousarray(synth.decode(b, dt).T) if tb else synth.decode(b, dt)
    a_st, b_st = synth.encode(a_st, dt), synth.encode(b_st, dt)
    out = empty((M, N), dt)
    hip.matmul(to_device(a_st, dt), to_device(b_st, dt), out, M, K, N, bool(ta), bool(tb))
    ref = orc.matmul(a, b, dt)
    assert_close(to_host(out, dt), ref, dt, what=f"matmul {M}x{K}x{N} t{ta}{tb}")


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("bcast_b", [True, False])
def test_batched_matmul(hip, orc, dt, bcast_b):
    batch, M, K, N = 3, 33, 40, 24
    a = rand((batch, M, K), dt, 3)
    b = rand((batch, K, N) if not bcast_b else (K, N), dt, 4)
    out = empty((batch, M, N), dt)
    hip.batched_matmul(to_device(a, dt), to_device(b, dt), out, batch, M, K, N, False, False, M * K,
                       0 if bcast_b else K * N, M * N)
    ref = orc.matmul(a, b, dt)
    assert_close(to_host(out, dt), ref, dt, what="batched_matmul")


def test_matmul_closed_form(hip):
    """all-ones known answer (reference tests/unified_tests.cpp:50-64): every entry == K."""
    for dt in DTS:
        M, K, N = 17, 96, 33
        a, b = synth.encode(np.ones((M, K)), dt), synth.encode(np.ones((K, N)), dt)
        out = empty((M, N), dt)
        hip.matmul(to_device(a, dt), to_device(b, dt), out, M, K, N)
        assert np.all(dec(to_host(out, dt), dt) == K)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("resid", [False, True])
@pytest.mark.parametrize("has_bias", [True, False])
def test_linear_fused(hip, orc, dt, act, resid, has_bias):
    M, K, N = 96, 160, 72
    x, w = rand((M, K), dt, 5), rand((K, N), dt, 6, 0.2)
    bias = rand((N,), dt, 7) if has_bias else None
    r = rand((M, N), dt, 8)
    ref = orc.linear(x, w, bias, dt)
    if act == 1:
        ref = orc.relu(ref, dt)
    elif act == 2:
        ref = orc.gelu(ref, dt)
    if resid:
        ref = orc.add(r, ref, dt)
    wd = to_device(w, dt)
    wt = empty((N, K), dt)
    hip.pack_linear_weight(wd, wt, K, N)
    out = empty((M, N), dt)
    hip.linear(to_device(x, dt), wt, to_device(bias, dt) if has_bias else None, out, M, K, N, act,
               to_device(r, dt) if resid else None)
    assert_close(to_host(out, dt), ref, dt, what=f"linear act={act} resid={resid} bias={has_bias}")


def _mha_params(E, dt, seed):
    p = {}
    for i, n in enumerate(("q_proj", "k_proj", "v_proj", "out_proj")):
        p[n + ".weight"] = rand((E, E), dt, seed + i, 1.0 / np.sqrt(E))
        p[n + ".bias"] = rand((E,), dt, seed + 10 + i, 0.1)
    return p


@pytest.mark.parametrize("dt", [F16, BF16, F32])
@pytest.mark.parametrize("B,T,E,H", [(2, 40, 64, 2), (1, 3, 8, 2), (3, 20, 48, 3), (1, 16, 40, 2), (1, 17, 96, 6),
                                     (2, 9, 96, 2), (2, 1024, 768, 12)])
def test_qkv_headsplit_bits(hip, dt, B, T, E, H):
    """The head-split projection stores exactly the bits of the row-major
    Linear with the concatenated weight, each column at [which][b, h, t, d]:
    head widths below 16 and sequences below 16 take the per-element index
    divisions, the rest the stepped column and row offsets (heads of 16, 20,
    32 and 64 columns; the decoder's shape on its 128x288 tile)."""
    hd = E // H
    x = rand((B * T, E), dt, 120)
    w = rand((E, 3 * E), dt, 121, 1.0 / np.sqrt(E))
    b = rand((3 * E,), dt, 122, 0.1)
    wt = empty((3 * E, E), dt)
    hip.pack_linear_weight(to_device(w, dt), wt, E, 3 * E)
    xd, bd = to_device(x, dt), to_device(b, dt)
    flat = empty((B * T, 3 * E), dt)
    hip.linear(xd, wt, bd, flat, B * T, E, 3 * E)
    q, k, v = (empty((B * H * T * hd,), dt) for _ in range(3))
    hip.qkv_projection(xd, wt, bd, q, k, v, B, T, E, H)
    ref = to_host(flat, dt).reshape(B, T, 3, H, hd).transpose(2, 0, 3, 1, 4)
    for i, t in enumerate((q, k, v)):
        assert np.array_equal(to_host(t, dt).reshape(B, H, T, hd), ref[i]), "qkv"[i]


@pytest.mark.parametrize("dt", [F16, BF16, F32])
@pytest.mark.parametrize("B,T,H,hd", [(2, 64, 2, 64), (1, 200, 3, 64), (64, 72, 4, 64), (1, 77, 2, 64),
                                      (2, 40, 2, 32), (1, 3, 2, 4),
                                      (1, 128, 2, 64), (2, 192, 3, 64), (1, 320, 2, 64), (5, 256, 16, 64),
                                      (1, 384, 47, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_core(hip, orc, dt, B, T, H, hd, causal):
    """q/k/v projection (fused head split) + fused attention vs the reference
    MHA core, including MuNet's K-reinterpretation.  hd = 64 with T % 8 == 0
    runs the pre-transposed-operand kernel (T = 72 with 256 (b,h) blocks takes
    its 32-rows-per-wave variant and a ragged last tile); T = 77 runs the
    in-LDS-transpose kernel; the rest the generic kernel."""
    E = H * hd
    x = rand((B * T, E), dt, 20)
    p = _mha_params(E, dt, 30)
    q2 = orc.linear(x, p["q_proj.weight"], p["q_proj.bias"], dt)
    k2 = orc.linear(x, p["k_proj.weight"], p["k_proj.bias"], dt)
    v2 = orc.linear(x, p["v_proj.weight"], p["v_proj.bias"], dt)
    ref = orc.mha_core(q2, k2, v2, B, T, H, causal, dt)
    # device: packed [3E, E] weight, head-split projection, attention
    w_cat = np.concatenate([p["q_proj.weight"], p["k_proj.weight"], p["v_proj.weight"]], axis=1)  # [E, 3E]
    b_cat = np.concatenate([p["q_proj.bias"], p["k_proj.bias"], p["v_proj.bias"]])
    wd = to_device(w_cat, dt)
    wt = empty((3 * E, E), dt)
    hip.pack_linear_weight(wd, wt, E, 3 * E)
    q, k, v = (empty((B * H * T * hd,), dt) for _ in range(3))
    hip.qkv_projection(to_device(x, dt), wt, to_device(b_cat, dt), q, k, v, B, T, E, H)
    ctx = empty((B * T, E), dt)
    hip.attention(q, k, v, ctx, B, H, T, hd, causal)
    assert_close(to_host(ctx, dt), ref, dt, what="attention")


@pytest.mark.parametrize("dt", [F16, BF16])
@pytest.mark.parametrize("B,T,H", [(4, 1024, 12), (1, 128, 2), (2, 192, 3), (5, 256, 16), (1, 384, 47), (8, 256, 8)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_pipelined_kernel_bits(hip, dt, B, T, H, causal, monkeypatch):
    """The software-pipelined flash kernel (T % 64 == 0) gives the bits of the
    single-trip kernel it replaces, in both work orders, at the decoder's full
    size and over the trip remainders (1-6 and 16 key tiles) and partial
    second rounds of the CU-paired order."""
    hd = 64
    q, k, v = (to_device(rand((B * H * T * hd,), dt, 70 + i, 0.5), dt) for i in range(3))
    outs = {}
    for name, env in (("pipe", {}), ("pipe_plain_order", {"MUNET_HIP_ATTN_ORDER": "0"}),
                      ("tr", {"MUNET_HIP_ATTN_KERNEL": "tr"})):
        monkeypatch.delenv("MUNET_HIP_ATTN_ORDER", raising=False)
        monkeypatch.delenv("MUNET_HIP_ATTN_KERNEL", raising=False)
        for key, val in env.items():
            monkeypatch.setenv(key, val)
        ctx = empty((B * T, H * hd), dt)
        hip.attention(q, k, v, ctx, B, H, T, hd, causal)
        hip.synchronize()
        outs[name] = to_host(ctx, dt)
    assert np.all(np.isfinite(dec(outs["pipe"], dt)))
    for name in ("pipe_plain_order", "tr"):
        assert np.array_equal(outs["pipe"], outs[name]), f"pipelined kernel differs from {name}"


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("rows,cols", [(64, 768), (33, 512), (5, 100), (3, 2000), (17, 1024), (9, 136), (20, 8)])
def test_layer_norm(hip, orc, dt, rows, cols):
    """16-bit rows with cols % 8 == 0 up to 1024 take the 16-lane kernel
    (ragged chunk counts: 136 / 8 = 17 chunks over 16 lanes), the rest the
    one-wave kernels."""
    x, w, b = rand((rows, cols), dt, 40, 3.0), rand((cols,), dt, 41), rand((cols,), dt, 42)
    out = empty((rows, cols), dt)
    hip.layer_norm(to_device(x, dt), to_device(w, dt), to_device(b, dt), out, rows, cols, 1e-5)
    assert_close(to_host(out, dt), orc.layer_norm(x, w, b, dt), dt, what="layer_norm")


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("rows,cols", [(64, 10), (17, 1000), (4, 3)])
def test_softmax(hip, orc, dt, rows, cols):
    x = rand((rows, cols), dt, 50, 4.0)
    out = empty((rows, cols), dt)
    hip.softmax(to_device(x, dt), out, rows, cols)
    assert_close(to_host(out, dt), orc.softmax(x, dt), dt, what="softmax")


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("op", [ADD, SUB, MUL, DIV])
@pytest.mark.parametrize("sa,sb", [((4, 5, 6), (4, 5, 6)), ((7, 9), (9,)), ((3, 1, 5), (1, 4, 1)), ((6,), (2, 3, 6))])
def test_binary_broadcast(hip, orc, dt, op, sa, sb):
    a = rand(sa, dt, 60)
    b = rand(sb, dt, 61)
    if op == DIV:
        b = synth.encode(np.abs(dec(b, dt)) + 0.5, dt)
    out_shape, stra, strb = compute_broadcast(sa, contiguous_strides(sa), sb, contiguous_strides(sb))
    out = empty(out_shape, dt)
    fn = {ADD: hip.add, SUB: hip.sub, MUL: hip.mul, DIV: hip.div}[op]
    fn(to_device(a, dt), to_device(b, dt), out, BroadcastInfo(out_shape, stra, strb))
    assert_close(to_host(out, dt), orc.binary(op, a, b, dt), dt, what=f"binary op={op}")


@pytest.mark.parametrize("dt", DTS)
def test_unary(hip, orc, dt):
    x = rand((1000,), dt, 70, 3.0)
    for name in ("relu", "sigmoid", "gelu"):
        out = empty((1000,), dt)
        getattr(hip, name)(to_device(x, dt), out, 1000)
        ref = getattr(orc, name)(x, dt)
        if name == "relu":
            assert np.array_equal(to_host(out, dt), ref)
        else:
            assert_close(to_host(out, dt), ref, dt, what=name)


@pytest.mark.parametrize("dt", DTS)
def test_elementwise_vector_path_bits(hip, dt):
    """Whole 16-byte chunks of contiguous operands take the vectorised
    kernels; the same values one element off a 16-byte boundary take the
    scalar ones: bit for bit the same for every unary op and the four binary
    ops (and the 1003-element tail case through the scalar kernel)."""
    n = 4096
    x = rand((n,), dt, 71, 2.0)
    y = synth.encode(np.abs(dec(rand((n,), dt, 72, 2.0), dt)) + 0.5, dt)
    # the same values at element 0 (aligned) and at element 1 (misaligned)
    dev = {off: (to_device(np.concatenate([x[:off], x]), dt), to_device(np.concatenate([y[:off], y]), dt))
           for off in (0, 1)}
    for name in ("relu", "sigmoid", "gelu"):
        outs = []
        for off in (0, 1):
            out = empty((n + off,), dt)
            getattr(hip, name)(dev[off][0][off:], out[off:], n)
            outs.append(to_host(out, dt)[off:])
        assert np.array_equal(outs[0], outs[1]), name
    info = BroadcastInfo((n,), (1,), (1,))
    for fn in (hip.add, hip.sub, hip.mul, hip.div):
        outs = []
        for off in (0, 1):
            out = empty((n + off,), dt)
            fn(dev[off][0][off:], dev[off][1][off:], out[off:], info)
            outs.append(to_host(out, dt)[off:])
        assert np.array_equal(outs[0], outs[1])
    xt = rand((1003,), dt, 73, 3.0)
    out = empty((1003,), dt)
    hip.relu(to_device(xt, dt), out, 1003)
    assert np.array_equal(to_host(out, dt), np.where(dec(xt, dt) > 0, xt, synth.encode(np.zeros(1003), dt)))


def test_gelu_known_values(hip):
    """x*sigmoid(1.702x) at -2, 0, 2 (reference tests/test_nn.cpp:385-402)."""
    x = synth.encode(np.array([-2.0, 0.0, 2.0]), F32)
    out = empty((3,), F32)
    hip.gelu(to_device(x, F32), out, 3)
    np.testing.assert_allclose(to_host(out, F32), [-0.0643, 0.0, 1.9357], atol=5e-3)


@pytest.mark.parametrize("dt", DTS)
def test_masked_fill(hip, orc, dt):
    n = 513
    x = rand((n,), dt, 80)
    mask = (np.arange(n) % 3 == 0).astype(np.int32)
    out = empty((n,), dt)
    hip.masked_fill(to_device(x, dt), to_device(mask, I32), out, n, -1e9)
    assert np.array_equal(to_host(out, dt), orc.masked_fill(x, mask, -1e9, dt))


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("D", [24, 30, 136, 768, 1024, 1100])
def test_embedding(hip, orc, dt, D):
    """16-bit rows with D % 8 == 0 up to 1024 take the 16-lane kernel, other
    rows with D % 4 == 0 up to 1024 the one-wave vector kernel, the rest the
    scalar one.  A -0.0 in the table keeps its sign without a position table."""
    V, B, T = 50, 3, 7
    w = rand((V, D), dt, 90)
    w[:, 1] = synth.encode(np.array([-0.0]), dt)[0]
    ids = np.random.default_rng(1).integers(0, V, (B, T)).astype(np.int32)
    out = empty((B * T, D), dt)
    hip.embedding(to_device(ids, I32), to_device(w, dt), out, B * T, V, D)
    assert np.array_equal(to_host(out, dt).reshape(B, T, D), orc.embedding(ids, w, dt))
    # fused token + position embedding == gather + gather + add
    pos = rand((T, D), dt, 91)
    out2 = empty((B * T, D), dt)
    hip.embedding_pos(to_device(ids, I32), to_device(w, dt), to_device(pos, dt), out2, B * T, V, D, T)
    ref = orc.add(orc.embedding(ids, w, dt), orc.embedding(np.tile(np.arange(T, dtype=np.int32), (B, 1)), pos, dt), dt)
    assert np.array_equal(to_host(out2, dt).reshape(B, T, D), ref)


def test_embedding_out_of_range(hip):
    from munet_amd._lib import HipError
    w = rand((10, 8), F32, 92)
    ids = np.array([1, 10, 3], dtype=np.int32)
    out = empty((3, 8), F32)
    hip.embedding(to_device(ids, I32), to_device(w, F32), out, 3, 10, 8)
    with pytest.raises(HipError, match="Embedding index out of range"):
        hip.check_device_errors()
    hip.check_device_errors()  # flag cleared


@pytest.mark.parametrize("dt", DTS)
def test_argmax(hip, dt):
    rows, cols = 40, 3000
    x = rand((rows, cols), dt, 93)
    x[5, 17] = x[5, 2000] = synth.encode(np.array([50.0]), dt)[0]  # tie -> first index
    out = empty((rows,), I32)
    hip.argmax(to_device(x, dt), out, rows, cols)
    assert np.array_equal(to_host(out, I32), np.argmax(dec(x, dt), axis=1))


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("B,iC,H,W,oC,k,s,p", [(2, 3, 9, 9, 4, 3, 1, 1), (2, 3, 9, 9, 4, 3, 2, 1),
                                               (1, 16, 12, 10, 32, 3, 1, 1), (2, 8, 8, 8, 16, 1, 1, 0),
                                               (1, 32, 16, 16, 16, 3, 2, 1),
                                               # whole 64-channel slabs: the pipelined implicit GEMM (16-bit)
                                               (2, 64, 12, 10, 32, 3, 1, 1), (1, 128, 9, 9, 64, 3, 2, 1),
                                               (1, 64, 8, 8, 2, 1, 1, 0), (2, 192, 7, 5, 96, 3, 1, 1),
                                               # 1x1 to few channels: the per-pixel dot-product kernel
                                               (3, 128, 10, 9, 6, 1, 1, 0), (1, 512, 4, 4, 1, 1, 1, 0)])
def test_conv2d(hip, orc, dt, B, iC, H, W, oC, k, s, p):
    x = rand((B, iC, H, W), dt, 100)
    w = rand((oC, iC, k, k), dt, 101, np.sqrt(2.0 / (iC * k * k)))
    b = rand((oC,), dt, 102, 0.1)
    ref = orc.conv2d(x, w, b, s, p, dt)
    out = empty(ref.shape, dt)
    hip.conv2d(to_device(x, dt), to_device(w, dt), to_device(b, dt), out, B, iC, H, W, oC, k, k, s, p)
    assert_close(to_host(out, dt), ref, dt, what="conv2d")


@pytest.mark.parametrize("dt", [F16, BF16])
@pytest.mark.parametrize("B,iC,H,W,oC,k,s,p,act", [(8, 64, 32, 32, 64, 3, 1, 1, 1), (2, 128, 16, 16, 256, 3, 2, 1, 1),
                                                   (1, 512, 8, 8, 512, 3, 1, 1, 1), (4, 64, 20, 12, 128, 3, 1, 1, 0),
                                                   (3, 256, 9, 7, 64, 3, 2, 1, 1), (2, 64, 16, 16, 16, 1, 1, 0, 0),
                                                   (1, 64, 5, 6, 40, 5, 1, 2, 1)])
def test_conv_pipelined_kernel_bits(hip, dt, B, iC, H, W, oC, k, s, p, act, monkeypatch):
    """The pipelined implicit-GEMM convolutions (iC % 64 == 0) give the bits
    of the general implicit-GEMM kernel (same MFMA sequence, bias added to the
    fp32 accumulator, one rounding, ReLU) on NHWC inputs, over the block
    tiles (the automatic choice, the register-staged 32x64 / 64x32 tiles and
    the direct-to-LDS 64x64 four / three stages, 32x64 four stages, 64x128
    three stages, and the eight-wave 128x64, 256x64 and 128x128 forced),
    strides, 1x1 and 5x5 filters, ragged pixel
    counts and padding on every side (the direct-to-LDS loads of padding
    taps read past the buffer resource and land as zeros)."""
    x = rand((B, H, W, iC), dt, 120)
    w = rand((oC, iC, k, k), dt, 121, np.sqrt(2.0 / (iC * k * k)))
    b = rand((oC,), dt, 122, 0.1)
    oh, ow = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    wo = empty((oC, k, k, iC), dt)
    hip.pack_conv_weight(to_device(w, dt), wo, oC, iC, k, k)
    xd, bd = to_device(x, dt), to_device(b, dt)
    outs = {}
    tiles = ("pipelined",) + tuple(f"tile{t}" for t in range(3, 12))
    for name in tiles + ("general",):
        monkeypatch.delenv("MUNET_HIP_CONV_KERNEL", raising=False)
        monkeypatch.delenv("MUNET_HIP_CONV_TILE", raising=False)
        if name == "general":
            monkeypatch.setenv("MUNET_HIP_CONV_KERNEL", "general")
        elif name.startswith("tile"):
            monkeypatch.setenv("MUNET_HIP_CONV_TILE", name[4:])
        out = empty((B, oh, ow, oC), dt)
        hip.conv2d_nhwc(xd, wo, bd, out, B, iC, H, W, oC, k, k, s, p, act)
        hip.synchronize()
        outs[name] = to_host(out, dt)
    assert np.all(np.isfinite(dec(outs["pipelined"], dt)))
    for name in tiles:
        assert np.array_equal(outs[name], outs["general"]), f"{name} conv differs from the general kernel"


def test_conv2d_closed_form(hip):
    """all-ones 3x3 conv, pad 0: every output == iC*9 (unified_tests.cpp:66-82)."""
    B, iC, H, W, oC = 1, 4, 6, 6, 8
    x = synth.encode(np.ones((B, iC, H, W)), F32)
    w = synth.encode(np.ones((oC, iC, 3, 3)), F32)
    out = empty((B, oC, 4, 4), F32)
    hip.conv2d(to_device(x, F32), to_device(w, F32), None, out, B, iC, H, W, oC, 3, 3, 1, 0)
    assert np.all(to_host(out, F32) == iC * 9)


@pytest.mark.parametrize("dt", [F16, BF16, F32])
def test_conv_transpose2d(hip, orc, dt):
    from oracle.models import conv_transpose2d
    B, iC, H, W, oC = 2, 16, 5, 6, 8
    x = rand((B, iC, H, W), dt, 110)
    w = rand((iC, oC, 2, 2), dt, 111, 0.3)
    b = rand((oC,), dt, 112, 0.1)
    ref = conv_transpose2d(orc, x, w, b, 2, dt)
    xd = to_device(x, dt)
    xn = empty((B, H, W, iC), dt)
    hip.nchw_to_nhwc(xd, xn, B, iC, H * W)
    wp = empty((4 * oC, iC), dt)
    hip.pack_convt_weight(to_device(w, dt), wp, iC, oC, 2)
    on = empty((B, 2 * H, 2 * W, oC), dt)
    hip.conv_transpose2d_nhwc(xn, wp, to_device(b, dt), on, B, iC, H, W, oC, 2)
    out = empty((B, oC, 2 * H, 2 * W), dt)
    hip.nhwc_to_nchw(on, out, B, oC, 4 * H * W)
    assert_close(to_host(out, dt), ref, dt, what="conv_transpose2d")


@pytest.mark.parametrize("dt", [F16, BF16])
@pytest.mark.parametrize("B,iC,H,W,oC", [(8, 128, 32, 32, 64), (2, 512, 8, 8, 256), (3, 64, 5, 7, 12)])
def test_conv_transpose_pipelined_epilogue_bits(hip, dt, B, iC, H, W, oC, monkeypatch):
    """The pipelined kernel's register epilogue for the transposed-conv
    scatter (row and column parts of the output offset, bias of column
    n mod oC) gives the bits of the general kernel's staged store, including
    a ragged tile and 12 output channels."""
    x = rand((B, H, W, iC), dt, 130)
    w = rand((iC, oC, 2, 2), dt, 131, 0.3)
    b = rand((oC,), dt, 132, 0.1)
    wp = empty((4 * oC, iC), dt)
    hip.pack_convt_weight(to_device(w, dt), wp, iC, oC, 2)
    xd, bd = to_device(x, dt), to_device(b, dt)
    outs = {}
    for name in ("pipelined", "general"):
        monkeypatch.delenv("MUNET_HIP_GEMM_TILE", raising=False)
        if name == "general":
            monkeypatch.setenv("MUNET_HIP_GEMM_TILE", "104")
        on = empty((B, 2 * H, 2 * W, oC), dt)
        hip.conv_transpose2d_nhwc(xd, wp, bd, on, B, iC, H, W, oC, 2)
        hip.synchronize()
        outs[name] = to_host(on, dt)
    assert np.array_equal(outs["pipelined"], outs["general"]), "pipelined transposed conv differs from the general kernel"


@pytest.mark.parametrize("dt", DTS)
def test_pool_upsample_concat(hip, orc, dt):
    B, C, H, W = 2, 3, 8, 6
    x = rand((B, C, H, W), dt, 120)
    xd = to_device(x, dt)
    out = empty((B, C, 4, 3), dt)
    hip.max_pool2d(xd, out, B, C, H, W, 2, 2, 0)
    assert np.array_equal(to_host(out, dt), orc.max_pool2d(x, 2, 2, 0, dt))
    out = empty((B, C, 3, 2), dt)
    hip.max_pool2d(xd, out, B, C, H, W, 3, 3, 1)
    assert np.array_equal(to_host(out, dt), orc.max_pool2d(x, 3, 3, 1, dt))
    up = empty((B, C, 2 * H, 2 * W), dt)
    hip.upsample2d(xd, up, B, C, H, W, 2)
    assert np.array_equal(to_host(up, dt), orc.upsample2d(x, 2, dt))
    y = rand((B, 5, H, W), dt, 121)
    cat = empty((B, C + 5, H, W), dt)
    hip.concat([xd, to_device(y, dt)], cat, 1, [x.shape, y.shape])
    assert np.array_equal(to_host(cat, dt), np.concatenate([x, y], axis=1))
    # NHWC variants agree with NCHW after a layout change
    xn = empty((B, H, W, C), dt)
    hip.nchw_to_nhwc(xd, xn, B, C, H * W)
    pn = empty((B, 4, 3, C), dt)
    hip.max_pool2d_nhwc(xn, pn, B, C, H, W, 2, 2, 0)
    assert np.array_equal(to_host(pn, dt).transpose(0, 3, 1, 2), orc.max_pool2d(x, 2, 2, 0, dt))
    un = empty((B, 2 * H, 2 * W, C), dt)
    hip.upsample2d_nhwc(xn, un, B, C, H, W, 2)
    assert np.array_equal(to_host(un, dt).transpose(0, 3, 1, 2), orc.upsample2d(x, 2, dt))


@pytest.mark.parametrize("dt", DTS + [I32])
def test_to_contiguous(hip, dt):
    x = rand((4, 5, 6), dt, 130) if dt != I32 else np.arange(120, dtype=np.int32).reshape(4, 5, 6)
    xd = to_device(x, dt)
    out = empty((6, 4, 5), dt)
    # permute(2,0,1) view of the contiguous [4,5,6] storage, offset 0
    hip.to_contiguous(xd, out, [6, 4, 5], [1, 30, 6], 0)
    assert np.array_equal(to_host(out, dt), np.ascontiguousarray(x.transpose(2, 0, 1)))
    out2 = empty((3, 5), dt)
    hip.to_contiguous(xd, out2, [3, 5], [30, 6], 7)  # narrow with an offset
    flat = x.reshape(-1)
    ref = np.array([[flat[7 + 30 * i + 6 * j] for j in range(5)] for i in range(3)])
    assert np.array_equal(to_host(out2, dt), ref)


def test_fast_f16_rounding_is_exhaustively_exact(hip):
    """The kernels' fast fp16 rounding (a bit trick for zero and the normal
    half range, the codec for the rest) equals the full codec, which
    test_convert_codecs pins to the reference, on all 2^32 float bit
    patterns: ties, half subnormals, overflow to infinity, NaN, signed zero."""
    assert hip.check_f16_rounding() == 0


def test_convert_codecs(hip, orc):
    vals = np.random.default_rng(5).standard_normal(4096).astype(np.float32) * 1000
    vals[:6] = [65519.0, 65520.0, 1e-8, -1e9, 0.5 + 2 ** -12, 3.0e-5]
    xd = to_device(vals, F32)
    for dt in (F16, BF16):
        out = empty((4096,), dt)
        hip.convert(xd, out, 4096)
        assert np.array_equal(to_host(out, dt), orc.encode(vals, dt))
