"""Engine caller features on the GPU: per-shape instances under a wildcard
contract, the prepared-input cache, run_batch, the observer's run events, the
pinned-host staging path and engines built from deploy artifacts (reference
src/inference.hpp:31-289, 538-627), each checked against the CPU oracle (the
restatement of MuNet's CPU backend, or MuNet's own compiled loader and
forward for the artifacts) and bit-exactly against plain runs of an engine
compiled for that exact shape."""
import numpy as np
import pytest

from munet_amd import models, synth
from munet_amd.engine import Engine
from oracle import CpuOracle, available
from oracle import models as omodels
from util import assert_close

pytestmark = pytest.mark.gpu


def _vs_oracle(orc, cfg, p, x, y, what):
    dt = synth.DTYPE_CODES[cfg.get("dtype", "float32")]
    assert_close(y, omodels.forward(orc, cfg, p, x), dt, what=what)


def _mlp():
    cfg = models.mlp_config()
    return cfg, models.init_params(cfg, "mlp", scope="feat")


def _x(cfg, b, scope):
    return models.make_input(cfg, (b, 784), "mlp", scope=scope)


def test_wildcard_batch_matches_exact_engines(orc):
    cfg, p = _mlp()
    e = Engine(0).load(cfg, p).compile((8, 784), expected_input_shape=(-1, 784))
    for b in (8, 16, 3, 16):
        x = _x(cfg, b, f"w{b}")
        ref = Engine(0).load(cfg, p).compile((b, 784)).run(x)
        y = e.run(x)
        assert np.array_equal(y, ref)
        _vs_oracle(orc, cfg, p, x, y, f"wildcard batch {b}")
    assert e.stats()["compiled_instances"] == 3


def test_decoder_wildcard_batch(orc):
    cfg = models.decoder_config(vocab=500, ctx=64, d_model=64, num_heads=2, num_layers=2, ffn=128, dtype="bfloat16")
    p = models.init_params(cfg, "gpt", scope="featd")
    e = Engine(0).load(cfg, p).compile((2, 64), expected_input_shape=(-1, 64))
    for b in (1, 3):
        ids = models.make_input(cfg, (b, 64), "gpt", scope=f"featd{b}")
        y = e.run(ids)
        assert np.array_equal(y, Engine(0).load(cfg, p).compile((b, 64)).run(ids))
        _vs_oracle(orc, cfg, p, ids, y, f"decoder wildcard batch {b}")


def test_prepared_input_cache(orc):
    cfg, p = _mlp()
    e = Engine(0).load(cfg, p).compile((8, 784))
    x, x2 = _x(cfg, 8, "c1"), _x(cfg, 8, "c2")
    ref, ref2 = e.run(x), e.run(x2)
    _vs_oracle(orc, cfg, p, x, ref, "cached input")
    _vs_oracle(orc, cfg, p, x2, ref2, "cached input, new version")
    assert np.array_equal(e.run_prepared(x, key=1, version=0), ref)
    assert np.array_equal(e.run_prepared(x, key=1, version=0), ref)  # hit: no transfer
    st = e.stats()
    assert (st["prepared_input_cache_hits"], st["prepared_input_cache_misses"]) == (1, 1)
    # a new version of the same tensor is a miss and replaces the entry
    assert np.array_equal(e.run_prepared(x2, key=1, version=1), ref2)
    st = e.stats()
    assert st["prepared_input_cache_misses"] == 2 and st["prepared_input_cache_entries"] == 1
    # capacity 2: a third tensor evicts the oldest
    e.set_input_cache(2, 1 << 30)
    for k in (10, 11, 12):
        e.run_prepared(x, key=k)
    st = e.stats()
    assert st["prepared_input_cache_entries"] == 2 and st["prepared_input_cache_evictions"] == 1
    # entries larger than the byte budget are not cached
    e.set_input_cache(8, 16)
    e.run_prepared(x, key=20)
    assert e.stats()["prepared_input_cache_entries"] == 0


def test_run_batch_and_observer(orc):
    cfg, p = _mlp()
    e = Engine(0).load(cfg, p).compile((8, 784))
    xs = [_x(cfg, 8, f"b{i}") for i in range(3)]
    events = []
    e.set_observer(events.append)
    outs = e.run_batch(xs)
    for x, o in zip(xs, outs):
        _vs_oracle(orc, cfg, p, x, o, "run_batch")
        assert np.array_equal(o, e.run(x))
    kinds = [ev["type"] for ev in events[:6]]
    assert kinds == ["RunStarted", "RunCompleted"] * 3
    assert events[1]["output_shape"] == [8, 10] and events[1]["duration_ms"] > 0
    assert e.stats()["host_runs"] == 6


def test_pinned_io(orc):
    cfg = models.decoder_config(vocab=500, ctx=64, d_model=64, num_heads=2, num_layers=1, ffn=128, dtype="bfloat16")
    p = models.init_params(cfg, "gpt", scope="pin")
    ids = models.make_input(cfg, (2, 64), "gpt", scope="pin_in")
    e = Engine(0).load(cfg, p).compile((2, 64))
    ref = e.run(ids)
    pin_in, pin_out = e.pinned_io()
    pin_in[...] = ids
    e.run_pinned()
    assert np.array_equal(pin_out, ref)
    _vs_oracle(orc, cfg, p, ids, pin_out.copy(), "pinned-host forward")


@pytest.mark.skipif(not available("reference"), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("which", ["mlp_f32", "mlp_f16", "cnn_f32"])
def test_artifact_engine_vs_munet_loader(tmp_path, which):
    """An engine built from a deploy artifact against MuNet's own loader and
    forward on the same file (src/inference_serialization.cpp and the
    reference's CPU ops, compiled into oracle/_ref)."""
    from munet_amd.artifact import save_deploy_artifact
    cfg, scheme, shape = {"mlp_f32": (models.mlp_config(), "mlp", (64, 784)),
                          "mlp_f16": (models.mlp_config(dtype="float16"), "mlp", (64, 784)),
                          "cnn_f32": (models.cnn_config(), "he", (8, 3, 32, 32))}[which]
    p = models.init_params(cfg, scheme, scope="art_gpu")
    x = models.make_input(cfg, shape, scheme, scope="art_gpu_x")
    path = tmp_path / f"{which}.npz"
    save_deploy_artifact(str(path), cfg, p)
    y = Engine(0).load_artifact(str(path)).compile(shape).run(x)
    dt = synth.DTYPE_CODES[cfg["dtype"]]
    assert_close(y, CpuOracle("reference").load_forward(path, x, dt), dt, what=f"artifact {which} vs MuNet's loader")


def test_per_op_timings():
    """mh_engine_op_times (each op alone, replayed) and
    mh_engine_forward_op_times (each op inside the forward) list every op of
    the plan with its algorithmic work, and leave the engine's results
    unchanged; the in-forward times add up to one forward's graph time."""
    cfg = models.decoder_config(vocab=2000, ctx=256, d_model=256, num_heads=4, num_layers=2, ffn=1024,
                                dtype="bfloat16")
    p = models.init_params(cfg, "gpt", scope="optimes")
    ids = models.make_input(cfg, (4, 256), "gpt", scope="optimes_in")
    e = Engine(0).load(cfg, p).compile((4, 256))
    ref = e.run(ids)
    names = [o["name"] for o in e.plan()["ops"]]
    iso, fwd = e.op_times(3), e.forward_op_times(5)
    assert [o["name"] for o in iso] == names and [o["name"] for o in fwd] == names
    # in-forward times are differences of prefix-graph times: on this small
    # model an op's figure (a few us) is within the replay-to-replay noise, so
    # only their sum is checked against the graph time below
    for o in iso:
        assert o["us"] > 0
    for o in iso + fwd:
        if o["kind"] in ("gemm", "qkv_gemm", "attention"):
            assert o["flops"] > 0
    head = next(o for o in fwd if o["name"].startswith("head"))
    assert head["flops"] == 2.0 * 4 * 256 * 256 * 2000  # exact, not rounded to 6 digits
    assert [o["name"] for o in e.op_times(2, only=names[1])] == [names[1]]
    graph_ms = []
    for _ in range(5):
        e.run_device()
        graph_ms.append(e.stats()["last_forward_gpu_ms"])
    total_ms = sum(o["us"] for o in fwd) / 1e3
    assert 0.5 * min(graph_ms) < total_ms < 3.0 * min(graph_ms) + 0.05, (total_ms, graph_ms)
    assert np.array_equal(e.run(ids), ref)


@pytest.mark.parametrize("tile", [None, "209", "216", "217"])
def test_streamed_final_output_bit_identical(monkeypatch, tile):
    """A final output of at least 64 MiB (here 4 x 1024 x 32000 bf16 logits) is
    written by the head's epilogue with non-temporal stores: the same bits as
    ordinary stores (MUNET_HIP_STREAM_OUT=0), on the automatic tile and forced
    direct-to-LDS tiles (every fixed tile has the streamed program)."""
    if tile is not None:
        monkeypatch.setenv("MUNET_HIP_GEMM_TILE", tile)
    cfg = models.decoder_config(vocab=32000, ctx=1024, d_model=64, num_heads=2, num_layers=1, ffn=128,
                                dtype="bfloat16")
    p = models.init_params(cfg, "gpt", scope="nt")
    ids = models.make_input(cfg, (4, 1024), "gpt", scope="nt_in")
    e = Engine(0).load(cfg, p).compile((4, 1024))
    assert e.stats()["stream_out"]
    y = e.run(ids)
    assert np.array_equal(y, e.run(ids))
    monkeypatch.setenv("MUNET_HIP_STREAM_OUT", "0")
    e0 = Engine(0).load(cfg, p).compile((4, 1024))
    assert not e0.stats()["stream_out"]
    assert np.array_equal(y, e0.run(ids))


def test_measured_mfma_peak():
    """mh_measure_mfma_peak: a register-only loop of 16x16x32 MFMAs over the
    whole GPU lands between half and 1.2x the datasheet dense peak (2.5
    PFLOP/s bf16 and fp16) and rejects other dtypes."""
    from munet_amd import _lib
    from munet_amd.backend import HipBackend
    hip = HipBackend(0)
    for dt in (2, 1):
        f = hip.measure_mfma_peak(dt, 4000)
        assert 1.25e15 < f < 3.0e15, f
    with pytest.raises(_lib.HipError, match="dtype"):
        hip.measure_mfma_peak(0, 10)


def test_measured_hbm_read():
    """mh_measure_hbm_read: a read-only stream over 1 GiB lands between a
    quarter and 1.1x the datasheet 8 TB/s and rejects a buffer under 1 MiB."""
    import torch
    from munet_amd import _lib
    from munet_amd.backend import HipBackend
    hip = HipBackend(0)
    buf = torch.ones(1 << 29, device="cuda", dtype=torch.float16)
    r = hip.measure_hbm_read(buf, 3)
    assert 2.0e12 < r < 8.8e12, r
    with pytest.raises(_lib.HipError, match="at least 1 MiB"):
        hip.measure_hbm_read(buf[:1024], 1)


def test_engine_config_on_device(orc):
    """warmup_runs runs extra forwards at compile (compile_warmup_ms), a
    non-strict engine serves another batch size from its own instance, and
    every run event carries its own trace id."""
    cfg, p = _mlp()
    e = Engine(0).load(cfg, p).set_config(warmup_runs=3, strict_shape_check=False)
    events = []
    e.set_observer(events.append)
    e.compile((8, 784))
    assert e.stats()["compile_warmup_ms"] > 0
    x = _x(cfg, 8, "cfg8")
    y = e.run(x)
    _vs_oracle(orc, cfg, p, x, y, "warmed engine")
    x5 = _x(cfg, 5, "cfg5")
    _vs_oracle(orc, cfg, p, x5, e.run(x5), "non-strict engine, batch 5")
    runs = [ev for ev in events if ev["type"] == "RunStarted"]
    assert len(runs) == 2 and 0 < runs[0]["trace_id"] < runs[1]["trace_id"]
    assert e.stats()["last_run_trace_id"] == runs[1]["trace_id"]
