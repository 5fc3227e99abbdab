"""Write the golden vectors under tests/golden/ from MuNet's own CPU code.

Runs oracle/_ref/libmunet_ref.so (the reference's CPU sources compiled by
oracle/Makefile in this container) on small seeded inputs for the functions
only the reference itself can pin (MHA with its K reinterpretation, the
per-dtype rounding chains of matmul / Linear / GELU / softmax / LayerNorm,
fp16 masked_fill, the 3-D Linear path, conv / pool / upsample, embedding).
Each case is stored as inputs + expected output in one .npz (data only).

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from munet_amd import synth  # noqa: E402
from oracle import CpuOracle  # noqa: E402

DTS = {"f32": synth.F32, "f16": synth.F16, "bf16": synth.BF16}


def rnd(shape, dt, seed, scale=1.0):
    return synth.encode(np.random.default_rng(seed).standard_normal(shape) * scale, dt)


def cases(ref):
    for tag, dt in DTS.items():
        a, b = rnd((7, 13), dt, 1), rnd((13, 5), dt, 2)
        yield f"matmul_{tag}", dict(a=a, b=b, out=ref.matmul(a, b, dt))
        x3, w = rnd((2, 3, 6), dt, 3), rnd((6, 4), dt, 4)
        bias = rnd((4,), dt, 5)
        yield f"linear3d_{tag}", dict(x=x3, w=w, bias=bias, out=ref.linear(x3, w, bias, dt))
        g = rnd((64,), dt, 6, 3.0)
        yield f"gelu_{tag}", dict(x=g, out=ref.gelu(g, dt))
        s = rnd((4, 9), dt, 7, 3.0)
        yield f"softmax_{tag}", dict(x=s, out=ref.softmax(s, dt))
        lx, lw, lb = rnd((3, 10), dt, 8, 2.0), rnd((10,), dt, 9), rnd((10,), dt, 10)
        yield f"layer_norm_{tag}", dict(x=lx, w=lw, b=lb, out=ref.layer_norm(lx, lw, lb, dt))
        for causal in (0, 1):
            for (B, T, E, H) in ((1, 3, 4, 2), (2, 5, 8, 2)):
                x = rnd((B, T, E), dt, 11 + causal)
                p = {}
                for i, n in enumerate(("q_proj", "k_proj", "v_proj", "out_proj")):
                    p[n + ".weight"] = rnd((E, E), dt, 20 + i, 0.5)
                    p[n + ".bias"] = rnd((E,), dt, 30 + i, 0.1)
                out = ref.mha(x, p, H, causal, dt)
                yield f"mha_{tag}_c{causal}_B{B}T{T}E{E}H{H}", dict(x=x, heads=np.int32(H), causal=np.int32(causal),
                                                                   out=out, **{k.replace(".", "_"): v for k, v in p.items()})
        cx, cw, cb = rnd((2, 3, 6, 5), dt, 40), rnd((4, 3, 3, 3), dt, 41, 0.3), rnd((4,), dt, 42)
        yield f"conv2d_{tag}", dict(x=cx, w=cw, b=cb, out=ref.conv2d(cx, cw, cb, 1, 1, dt))
        yield f"conv2d_s2_{tag}", dict(x=cx, w=cw, b=cb, out=ref.conv2d(cx, cw, cb, 2, 1, dt))
        yield f"max_pool2d_{tag}", dict(x=cx, out=ref.max_pool2d(cx, 2, 2, 0, dt))
        yield f"upsample2d_{tag}", dict(x=cx, out=ref.upsample2d(cx, 2, dt))
        ids = np.random.default_rng(43).integers(0, 11, (2, 4)).astype(np.int32)
        ew = rnd((11, 6), dt, 44)
        yield f"embedding_{tag}", dict(ids=ids, w=ew, out=ref.embedding(ids, ew, dt))
        vals = np.array([65519.0, 65520.0, 1e-8, -1e9, 0.5 + 2 ** -12, 3.0e-5, -2.5, 1.0 + 2 ** -9], np.float32)
        yield f"encode_{tag}", dict(x=vals, out=ref.encode(vals, dt))


def main():
    ref = CpuOracle("reference")
    n = 0
    for name, arrays in cases(ref):
        np.savez(os.path.join(HERE, name + ".npz"), **arrays)
        n += 1
    print(f"wrote {n} golden cases to {HERE}")


if __name__ == "__main__":
    main()
