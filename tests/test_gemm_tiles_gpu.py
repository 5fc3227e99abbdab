"""Every GEMM block-tile variant (the general kernels of gemm.hip and
gemm_dma.hip, and the pipelined kernels: register-staged and direct-to-LDS,
128- and 256-row) against the oracle, forced through MUNET_HIP_GEMM_TILE (read
by the library at every GEMM call), on shapes with ragged M / N tails,
N % 4 != 0 (general epilogue), K from one to seven 64-wide slabs and ragged K
(short first slab; the direct-to-LDS tiles fall back to the register-staged
kernel there)."""
import pytest

from munet_amd import synth
from util import assert_close, rand

pytestmark = pytest.mark.gpu

SHAPES = [(300, 192, 200), (257, 128, 129), (64, 64, 64), (520, 256, 264), (96, 200, 72),
          (130, 320, 96), (70, 448, 136), (33, 40, 48), (530, 136, 392)]
TILES = [0, 1, 2, 3, 4, 5, 6, 100, 101, 102, 103, 104, 105, 106, 107, 200, 201, 202, 203, 207, 208, 209,
         210, 211, 212, 216, 217, 219]


@pytest.mark.parametrize("tile", TILES)
def test_forced_tile(tile, hip, orc, monkeypatch):
    from munet_amd.backend import empty, to_device, to_host
    monkeypatch.setenv("MUNET_HIP_GEMM_TILE", str(tile))
    for dt in (synth.BF16, synth.F16):
        for (M, K, N) in SHAPES:
            x, w, b = rand((M, K), dt, 1), rand((K, N), dt, 2, 0.2), rand((N,), dt, 3)
            r = rand((M, N), dt, 4)
            ref = orc.add(r, orc.gelu(orc.linear(x, w, b, dt), dt), dt)
            wt = empty((N, K), dt)
            hip.pack_linear_weight(to_device(w, dt), wt, K, N)
            out = empty((M, N), dt)
            hip.linear(to_device(x, dt), wt, to_device(b, dt), out, M, K, N, 2, to_device(r, dt))
            assert_close(to_host(out, dt), ref, dt, what=f"tile={tile} dt={dt} {M}x{K}x{N}")


@pytest.mark.parametrize("tile", [207, 208, 209, 210, 211, 212, 216, 217, 219])
def test_tiles_bit_identical_to_128(tile, hip, monkeypatch):
    """The 256-row and direct-to-LDS tiles accumulate every output in the
    same K order as the register-staged 128x128 tile (64-wide slabs, two
    32-wide MFMA halves), so their outputs are bit-identical, for every fused
    epilogue kind and the head split (K = 320: five slabs, so every stage
    count takes its unrolled loop and its tail)."""
    import torch
    from munet_amd.backend import empty
    g = torch.Generator(device="cuda").manual_seed(7)
    M, K, N = 520, 320, 392
    bf = torch.bfloat16
    x = torch.randn(M, K, device="cuda", generator=g).to(bf)
    wt = (torch.randn(N, K, device="cuda", generator=g) * 0.1).to(bf)
    bias = (torch.randn(N, device="cuda", generator=g) * 0.1).to(bf)
    r = torch.randn(M, N, device="cuda", generator=g).to(bf)
    for act, resid, use_bias in [(0, None, False), (0, None, True), (2, None, True), (1, None, True),
                                 (0, r, True), (0, r, False)]:
        outs = []
        for t in (200, tile):
            monkeypatch.setenv("MUNET_HIP_GEMM_TILE", str(t))
            out = empty((M, N), 2)
            hip.linear(x, wt, bias if use_bias else None, out, M, K, N, act, resid)
            torch.cuda.synchronize()
            outs.append(out.view(torch.int16).clone())
        assert torch.equal(outs[0], outs[1]), f"tile {tile} act={act} resid={resid is not None} bias={use_bias}"
    # head split: [B*T, 3E] -> q, k, v [B, H, T, hd]
    Bq, Tq, E, Hq = 2, 136, 192, 3
    xq = torch.randn(Bq * Tq, E, device="cuda", generator=g).to(bf)
    wq = (torch.randn(3 * E, E, device="cuda", generator=g) * 0.1).to(bf)
    bqk = (torch.randn(3 * E, device="cuda", generator=g) * 0.1).to(bf)
    res = []
    for t in (200, tile):
        monkeypatch.setenv("MUNET_HIP_GEMM_TILE", str(t))
        q, k, v = (empty((Bq * Tq * E,), 2) for _ in range(3))
        hip.qkv_projection(xq, wq, bqk, q, k, v, Bq, Tq, E, Hq)
        torch.cuda.synchronize()
        res.append(torch.cat([q, k, v]).view(torch.int16).clone())
    assert torch.equal(res[0], res[1]), f"tile {tile} head split"


@pytest.mark.parametrize("tile", [None, 200, 203, 208, 209, 216, 217])
def test_xcd_tile_enumeration_bit_identical(tile, hip, monkeypatch):
    """The per-XCD tile enumeration (row groups, or column groups of any width,
    a ragged last group included) only reorders the tiles: every output is
    computed by the same tile code, so the outputs are bit-identical.  Shapes
    have a tile count divisible by 8 (the enumeration applies) at 128x128,
    128x96 and 256x192; None is the automatic tile."""
    import torch
    from munet_amd.backend import empty
    if tile is not None:
        monkeypatch.setenv("MUNET_HIP_GEMM_TILE", str(tile))
    g = torch.Generator(device="cuda").manual_seed(9)
    bf = torch.bfloat16
    for (M, K, N) in [(1024, 192, 768), (512, 128, 1536), (256, 320, 3072), (2048, 64, 384)]:
        x = torch.randn(M, K, device="cuda", generator=g).to(bf)
        wt = (torch.randn(N, K, device="cuda", generator=g) * 0.1).to(bf)
        bias = (torch.randn(N, device="cuda", generator=g) * 0.1).to(bf)
        r = torch.randn(M, N, device="cuda", generator=g).to(bf)
        for act, resid in [(2, None), (0, r)]:
            outs = []
            for gn in ("0", "1", "3", "8", "16", "64"):
                monkeypatch.setenv("MUNET_HIP_XCD_GN", gn)
                out = empty((M, N), 2)
                hip.linear(x, wt, bias, out, M, K, N, act, resid)
                torch.cuda.synchronize()
                outs.append(out.view(torch.int16).clone())
            for gn, o in zip(("1", "3", "8", "16", "64"), outs[1:]):
                assert torch.equal(outs[0], o), f"tile {tile} gn {gn} {M}x{K}x{N} act={act}"


@pytest.mark.parametrize("tile", [200, 201, 202, 203, 208, 209, 216, 217])
def test_f16_fixed_programs_bit_identical_to_general(tile, hip, monkeypatch):
    """fp16 runs the fixed epilogue programs (plain, bias, bias+GELU,
    bias+ReLU, bias+residual) when the destination is 8-byte aligned; an
    output one element off that alignment takes the general program on the
    same tile.  Both round every step with MuNet's half-away fp16 codec, so the
    outputs are bit-identical."""
    import torch
    from munet_amd.backend import empty
    monkeypatch.setenv("MUNET_HIP_GEMM_TILE", str(tile))
    g = torch.Generator(device="cuda").manual_seed(11)
    M, K, N = 512, 320, 384
    h = torch.float16
    x = torch.randn(M, K, device="cuda", generator=g).to(h)
    wt = (torch.randn(N, K, device="cuda", generator=g) * 0.1).to(h)
    bias = (torch.randn(N, device="cuda", generator=g) * 0.1).to(h)
    r = torch.randn(M, N, device="cuda", generator=g).to(h)
    for act, resid, use_bias in [(0, None, False), (0, None, True), (2, None, True), (1, None, True), (0, r, True)]:
        outs = []
        for shift in (0, 1):
            buf = empty((M * N + 1,), 1)
            out = buf[shift:shift + M * N]
            hip.linear(x, wt, bias if use_bias else None, out, M, K, N, act, resid)
            torch.cuda.synchronize()
            outs.append(out.view(torch.int16).clone())
        assert torch.equal(outs[0], outs[1]), f"tile {tile} act={act} resid={resid is not None} bias={use_bias}"
