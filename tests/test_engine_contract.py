"""Engine shape contract with -1 wildcards (reference ShapeContract /
Engine::compile(example, expected_input_shape), src/inference.hpp:128-184,
446-537) and the observer events, on plan-only engines (no GPU)."""
import numpy as np
import pytest

from munet_amd import _lib, models, synth
from munet_amd.engine import Engine


def _zero_params(cfg):
    dt = synth.DTYPE_CODES[cfg.get("dtype", "float32")]
    return {n: np.zeros(s, dtype=synth.storage_dtype(dt)) for n, s, _r, _i in models.param_specs(cfg)}


def test_wildcard_batch_compiles_one_instance_per_shape():
    cfg = models.mlp_config()
    e = Engine(device=-1).load(cfg, _zero_params(cfg)).compile((8, 784), expected_input_shape=(-1, 784))
    assert e.out_shape == (8, 10)
    assert e.output_shape_for((16, 784)) == (16, 10)
    assert e.output_shape_for((3, 784)) == (3, 10)
    assert e.output_shape_for((16, 784)) == (16, 10)  # cached instance
    assert e.stats()["compiled_instances"] == 3


@pytest.mark.parametrize("shape,reason", [((16, 785), "dim mismatch at index 1"), ((16, 784, 1), "rank mismatch")])
def test_contract_rejects(shape, reason):
    cfg = models.mlp_config()
    e = Engine(device=-1).load(cfg, _zero_params(cfg)).compile((8, 784), expected_input_shape=(-1, 784))
    with pytest.raises(_lib.HipError, match=reason):
        e.output_shape_for(shape)


def test_exact_contract_rejects_other_batch():
    cfg = models.mlp_config()
    e = Engine(device=-1).load(cfg, _zero_params(cfg)).compile((8, 784))
    with pytest.raises(_lib.HipError, match="dim mismatch at index 0"):
        e.output_shape_for((9, 784))


def test_expected_shape_must_match_example():
    cfg = models.mlp_config()
    with pytest.raises(_lib.HipError, match="expected_input_shape mismatch"):
        Engine(device=-1).load(cfg, _zero_params(cfg)).compile((8, 784), expected_input_shape=(-1, 100))


def test_observer_compile_events():
    cfg = models.decoder_config(vocab=100, ctx=64, d_model=64, num_heads=2, num_layers=1, ffn=128)
    e = Engine(device=-1).load(cfg, _zero_params(cfg))
    events = []
    e.set_observer(events.append)
    e.compile((2, 64), expected_input_shape=(-1, 64))
    e.output_shape_for((4, 64))
    kinds = [ev["type"] for ev in events]
    # compile finishes the load first (reference Engine::load then compile)
    assert kinds == ["LoadStarted", "LoadCompleted", "CompileStarted", "CompileCompleted", "CompileStarted",
                     "CompileCompleted"]
    assert events[3]["output_shape"] == [2, 64, 100] and events[5]["input_shape"] == [4, 64]
    assert events[3]["duration_ms"] >= 0
    e.set_observer(None)
    e.output_shape_for((5, 64))
    assert len(events) == 6


def test_load_and_compile_events_with_trace_ids():
    """LoadStarted / LoadCompleted (parameter count in the message), then
    CompileStarted / CompileCompleted carrying a fresh trace id while an
    observer is attached (reference src/inference.hpp:393-537, 720-722)."""
    cfg = models.mlp_config()
    e = Engine(device=-1).load(cfg, _zero_params(cfg))
    events = []
    e.set_observer(events.append)
    e.finish_load()
    e.compile((8, 784))
    assert [ev["type"] for ev in events] == ["LoadStarted", "LoadCompleted", "CompileStarted", "CompileCompleted"]
    assert "6 parameter tensors" in events[1]["message"]
    assert events[2]["trace_id"] > 0 and events[2]["trace_id"] == events[3]["trace_id"]
    st = e.stats()
    assert st["last_compile_trace_id"] == events[2]["trace_id"]
    # without an observer, no trace id is drawn
    e2 = Engine(device=-1).load(cfg, _zero_params(cfg)).compile((8, 784))
    assert e2.stats()["last_compile_trace_id"] == 0


def test_engine_config():
    cfg = models.mlp_config()
    e = Engine(device=-1).load(cfg, _zero_params(cfg))
    with pytest.raises(_lib.HipError, match="warmup_runs must be >= 0"):
        e.set_config(warmup_runs=-1)
    events = []
    e.set_observer(events.append)
    e.set_config(warmup_runs=3, strict_shape_check=False, lean_mode=True)
    e.compile((8, 784))
    st = e.stats()
    assert st["warmup_runs"] == 3 and not st["strict_shape_check"] and st["lean_mode"]
    # lean mode: no parameter scan, no memory figures
    assert "parameter tensors" not in events[1]["message"]
    assert all(ev["current_memory_bytes"] == 0 for ev in events)
    # strict_shape_check off: another shape gets its own instance instead of
    # failing the compiled contract
    assert e.output_shape_for((9, 784)) == (9, 10)
    assert e.stats()["compiled_instances"] == 2
