"""Deploy-artifact loader (mh_engine_create_from_artifact) on plan-only
engines (no GPU): the reference's `munet_model` rev-1 .npz format and its
validations (src/inference_serialization.cpp:902-1080), bf16 tensors as <u2
bit patterns, and dtype conversion into the config's dtype."""
import json
import zipfile

import numpy as np
import pytest

from munet_amd import _lib, models, synth
from munet_amd.artifact import save_deploy_artifact
from munet_amd.engine import Engine
from oracle import CpuOracle, available


def _params(cfg, scheme):
    return models.init_params(cfg, scheme, scope="artifact")


def _decoder():
    return models.decoder_config(vocab=500, ctx=64, d_model=64, num_heads=2, num_layers=2, ffn=128,
                                 dtype="bfloat16")


def _plan_json(e):
    p = e.plan()
    return json.dumps(p["ops"], sort_keys=True), p["arena_bytes"]


@pytest.mark.parametrize("which", ["mlp", "decoder"])
def test_artifact_round_trip_plan(tmp_path, which):
    cfg, scheme, shape = ((models.mlp_config(), "mlp", (8, 784)) if which == "mlp"
                          else (_decoder(), "gpt", (2, 64)))
    params = _params(cfg, scheme)
    path = tmp_path / "model.npz"
    save_deploy_artifact(str(path), cfg, params)
    a = Engine(device=-1).load_artifact(str(path)).compile(shape)
    b = Engine(device=-1).load(cfg, params).compile(shape)
    assert _plan_json(a) == _plan_json(b)
    assert a.out_shape == b.out_shape
    assert a.config == cfg


def test_bf16_members_are_u2_bit_patterns(tmp_path):
    cfg = _decoder()
    params = _params(cfg, "gpt")
    path = tmp_path / "m.npz"
    save_deploy_artifact(str(path), cfg, params)
    with np.load(str(path), allow_pickle=False) as z:
        w = z["blocks.0.ff.0.weight"]
        assert w.dtype == np.dtype("<u2")
        assert np.array_equal(w, params["blocks.0.ff.0.weight"])
        assert json.loads(str(z["__tensor_names__"])) == sorted(params)


def _write(path, state):
    with open(path, "wb") as f:
        np.savez(f, **state)


def _good_state(cfg, params):
    """A minimal valid artifact's members (metadata the reference requires)."""
    state = dict(params)
    state.update({
        "__config__": np.array(json.dumps(cfg)),
        "__format_name__": np.array("munet_model"),
        "__format_revision__": np.array(1, dtype=np.int64),
        "__artifact_kind__": np.array("deploy_model"),
        "__artifact_scope__": np.array("runtime_only"),
        "__default_load_mode__": np.array("eval"),
        "__contains_training_state__": np.array(False),
        "__recommended_loader__": np.array("load_for_inference"),
        "__compile_contract_policy__": np.array("external"),
    })
    return state


@pytest.mark.parametrize("change,msg", [
    (lambda s: s.update(__format_name__=np.array("other")), "format name"),
    (lambda s: s.update(__format_revision__=np.array(2, dtype=np.int64)), "revision"),
    (lambda s: s.update(__artifact_kind__=np.array("training_checkpoint")), "artifact kind"),
    (lambda s: s.update(__artifact_scope__=np.array("training+inference")), "artifact scope"),
    (lambda s: s.update(__default_load_mode__=np.array("train")), "load mode"),
    (lambda s: s.update(__contains_training_state__=np.array(True)), "training state"),
    (lambda s: s.update(__recommended_loader__=np.array("load_checkpoint")), "recommended loader"),
    (lambda s: s.update(__compile_contract_policy__=np.array("dynamic")), "compile contract"),
    (lambda s: s.pop("__config__"), "__config__"),
    (lambda s: s.update({"optimizer.state": np.zeros(3, np.float32)}), "training state"),
    (lambda s: s.update(__tensor_names__=np.array(json.dumps(["a"]))), "manifest"),
    (lambda s: s.update(__producer__=np.array("someone_else")), "producer"),
    (lambda s: s.update({"0.weight": np.zeros((784, 256), np.float64)}), "unsupported dtype"),
])
def test_artifact_validation(tmp_path, change, msg):
    """Each malformed artifact is refused by this loader and, where the
    reference sources were built, by MuNet's own loader too."""
    cfg = models.mlp_config()
    state = _good_state(cfg, _params(cfg, "mlp"))
    change(state)
    path = tmp_path / "bad.npz"
    _write(path, state)
    with pytest.raises(_lib.HipError, match=msg):
        Engine(device=-1).load_artifact(str(path))
    if available("reference"):
        assert CpuOracle("reference").load_check(path) is not None, "MuNet's loader accepted it"


def test_compressed_members_are_rejected(tmp_path):
    cfg = models.mlp_config()
    path = tmp_path / "c.npz"
    with open(path, "wb") as f:
        np.savez_compressed(f, **_good_state(cfg, _params(cfg, "mlp")))
    with pytest.raises(_lib.HipError, match="compressed"):
        Engine(device=-1).load_artifact(str(path))


def test_not_a_zip(tmp_path):
    path = tmp_path / "x.npz"
    path.write_bytes(b"\x00" * 100)
    with pytest.raises(_lib.HipError, match="central directory"):
        Engine(device=-1).load_artifact(str(path))


def test_producer_must_be_munet(tmp_path):
    """The reference's deploy loader accepts exactly the producer tag 'munet'
    or none (src/inference_serialization.cpp:35, :997-1000); the tag its
    Python bindings write ('munet_nn', src/bindings.cpp:2049) is refused there
    too."""
    cfg = models.mlp_config()
    state = _good_state(cfg, _params(cfg, "mlp"))
    state["__producer__"] = np.array("munet")
    _write(tmp_path / "ok.npz", state)
    Engine(device=-1).load_artifact(str(tmp_path / "ok.npz")).compile((4, 784))
    for prod in ("munet_nn", "munetx", "munet_pytorch_interop"):
        state["__producer__"] = np.array(prod)
        path = tmp_path / f"{prod}.npz"
        _write(path, state)
        with pytest.raises(_lib.HipError, match="unsupported producer"):
            Engine(device=-1).load_artifact(str(path))


def test_zip64_members_parse(tmp_path):
    """numpy writes every member with ZIP64 local headers; check that is the
    layout under test and that it loads."""
    cfg = models.mlp_config()
    path = tmp_path / "z.npz"
    save_deploy_artifact(str(path), cfg, _params(cfg, "mlp"))
    with zipfile.ZipFile(path) as z:
        assert all(i.compress_type == zipfile.ZIP_STORED for i in z.infolist())
    Engine(device=-1).load_artifact(str(path)).compile((4, 784))


def _npy_bytes(descr, shape, payload):
    """A .npy member with a hand-written header (descr and shape as given)."""
    hdr = "{'descr': '%s', 'fortran_order': False, 'shape': %s, }" % (descr, shape)
    hdr += " " * ((64 - (10 + len(hdr) + 1) % 64) % 64) + "\n"
    return b"\x93NUMPY\x01\x00" + len(hdr).to_bytes(2, "little") + hdr.encode() + payload


@pytest.mark.parametrize("member,descr,shape,payload,msg", [
    # 2^62 UTF-32 characters: chars * 4 wraps to 0 in 64 bits
    ("__format_name__", "<U4611686018427387904", "()", b"m\0\0\0", "truncated"),
    ("__producer__", "|S18446744073709551615", "()", b"munet", "truncated"),
    # dimensions whose product wraps round to the payload's element count
    ("0.bias", "<f4", "(4294967296, 4294967296, 1)", b"\0" * 1024, "payload does not match|overflow"),
    ("0.bias", "<f4", "(256,)", b"\0" * 1023, "payload does not match"),
])
def test_malformed_npy_headers_are_rejected(tmp_path, member, descr, shape, payload, msg):
    """Header fields the parser must bound-check without overflowing: string
    lengths from the descr and the element count from the shape."""
    cfg = models.mlp_config()
    state = _good_state(cfg, _params(cfg, "mlp"))
    state["__producer__"] = np.array("munet")
    path = tmp_path / "bad.npz"
    with zipfile.ZipFile(path, "w", zipfile.ZIP_STORED) as z:
        for k, v in state.items():
            if k == member:
                z.writestr(k + ".npy", _npy_bytes(descr, shape, payload))
            else:
                import io
                buf = io.BytesIO()
                np.save(buf, v, allow_pickle=False)
                z.writestr(k + ".npy", buf.getvalue())
    with pytest.raises(_lib.HipError, match=msg):
        Engine(device=-1).load_artifact(str(path)).compile((4, 784))


needs_ref = pytest.mark.skipif(not available("reference"), reason="oracle/_ref not built (needs /root/reference)")


@needs_ref
@pytest.mark.parametrize("which", ["mlp_f32", "mlp_f16", "cnn_f32"])
def test_munet_loader_reads_our_artifacts(tmp_path, which):
    """MuNet's own deploy loader (src/inference_serialization.cpp, compiled
    into oracle/_ref) accepts the artifacts save_deploy_artifact writes, and
    the module it builds computes what the restatement computes from the
    parameter dict, bit for bit."""
    from oracle import models as om
    cfg, scheme, shape = {"mlp_f32": (models.mlp_config(), "mlp", (8, 784)),
                          "mlp_f16": (models.mlp_config(dtype="float16"), "mlp", (8, 784)),
                          "cnn_f32": (models.cnn_config(), "he", (2, 3, 32, 32))}[which]
    params = _params(cfg, scheme)
    x = models.make_input(cfg, shape, scheme, scope="art_x")
    path = tmp_path / f"{which}.npz"
    save_deploy_artifact(str(path), cfg, params)
    ref = CpuOracle("reference")
    assert ref.load_check(path) is None
    dt = synth.DTYPE_CODES[cfg["dtype"]]
    y = ref.load_forward(path, x, dt)
    assert np.array_equal(y, om.forward(CpuOracle("restatement"), cfg, params, x))


@needs_ref
def test_munet_loader_refuses_bf16_members(tmp_path):
    """MuNet's loader has no bf16 (src/inference_serialization.cpp:459-471);
    this loader takes bf16 members as <u2 bit patterns."""
    cfg = models.mlp_config(dtype="bfloat16")
    path = tmp_path / "bf16.npz"
    save_deploy_artifact(str(path), cfg, _params(cfg, "mlp"))
    assert CpuOracle("reference").load_check(path) is not None
    Engine(device=-1).load_artifact(str(path)).compile((4, 784))
