"""The real-checkpoint path on the CPU: an F32 model.safetensors (written here by the
`safetensors` package itself, an implementation independent of the library's reader) and its
config.json, exported to GGUF the way `t0-cli export-gguf` does (crates/cli/src/main.rs:283-295
-> Weights::load_bytes weights.rs:115-140 -> export_gguf weights.rs:184-227).

The export must be byte-identical to the oracle's export of the same F32 tensors (the oracle
restates weights.rs:184-227 from an F32 GGUF of them), at every quantization; the reader must
refuse what the safetensors crate refuses, non-F32 tensors (weights.rs:127-129) and configs
serde would not accept (config.rs:6-32)."""
import json
import struct

import numpy as np
import pytest
import safetensors.numpy

from test_oracle import _tensor_names
from util import TINY


@pytest.fixture(scope="module")
def checkpoint(t0hip, oracle):
    """A random-init model's F32 tensors as safetensors bytes, its config.json, and the oracle
    model of an F32 GGUF holding the same tensors."""
    cfg = dict(TINY, quantile_levels=(0.1, 0.25, 0.5, 0.75, 0.9))
    g = t0hip.synth_model_gguf(t0hip.make_config(**cfg), quant=0, seed=17)
    om = oracle.Model(g)
    tensors = {n: np.ascontiguousarray(om.tensor(n), np.float32) for n in _tensor_names(g)}
    st = safetensors.numpy.save(tensors, metadata={"format": "pt"})
    config = {"embed_dim": cfg["embed_dim"], "num_layers": cfg["num_layers"], "num_heads": cfg["num_heads"],
              "mlp_hidden_dim": cfg["mlp_hidden_dim"], "patch_size": cfg["patch_size"],
              "group_every_n": cfg["group_every_n"], "dropout": 0.0,
              "quantile_levels": [float(np.float32(q)) for q in cfg["quantile_levels"]],
              "scaler_use_arcsinh": True, "scaler_eps": float(np.float32(0.1)), "scaler_eps_mode": "variance_offset",
              "model_type": "t0"}  # serde ignores fields T0Config does not name
    return st, json.dumps(config), om, tensors


@pytest.mark.parametrize("quant", [8, 2, 1, 0])
def test_export_is_byte_identical_to_the_oracle(t0hip, checkpoint, quant):
    st, cj, om, _ = checkpoint
    assert t0hip.export_gguf_from_safetensors(st, cj, quant) == om.export_gguf(quant)


def test_config_defaults_and_beta_scaler(t0hip, checkpoint, oracle):
    """config.rs:24-32 defaults (arcsinh on, eps 0.1, variance_offset) when the keys are absent, and
    the beta scaler (std_clamp, eps 0.01) carried into the GGUF metadata."""
    st, cj, om, _ = checkpoint
    c = json.loads(cj)
    for k in ("scaler_use_arcsinh", "scaler_eps", "scaler_eps_mode"):
        c.pop(k)
    assert t0hip.export_gguf_from_safetensors(st, json.dumps(c), 8) == om.export_gguf(8)
    c.update(scaler_eps=0.01, scaler_eps_mode="std_clamp", scaler_use_arcsinh=False)
    cfg, _ = t0hip.inspect_gguf(t0hip.export_gguf_from_safetensors(st, json.dumps(c), 8))
    assert cfg.scaler_variance_offset == 0 and cfg.scaler_use_arcsinh == 0
    assert cfg.scaler_eps == np.float32(0.01)


def _status(t0hip, st, cj):
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.export_gguf_from_safetensors(st, cj, 8)
    return e.value.status, str(e.value)


def test_refuses_bad_safetensors(t0hip, checkpoint):
    st, cj, _, tensors = checkpoint
    n = struct.unpack_from("<Q", st, 0)[0]
    assert _status(t0hip, st[:5], cj)[0] == "SAFETENSORS"                       # header too small
    assert _status(t0hip, struct.pack("<Q", 2 ** 40) + st[8:], cj)[0] == "SAFETENSORS"  # header too large
    assert _status(t0hip, st[:8 + n // 2], cj)[0] == "SAFETENSORS"             # truncated header
    assert _status(t0hip, st[:-4], cj)[0] == "SAFETENSORS"                     # buffer not covered
    bad_json = st[:8] + b"{" + st[9:]
    bad_json = bad_json[:8 + n - 1] + b"x" + bad_json[8 + n:]
    assert _status(t0hip, bad_json, cj)[0] == "SAFETENSORS"
    # a non-F32 tensor (weights.rs:127-129)
    t16 = dict(tensors)
    t16["transformer.out_norm.scale"] = tensors["transformer.out_norm.scale"].astype(np.float16)
    status, msg = _status(t0hip, safetensors.numpy.save(t16), cj)
    assert status == "SAFETENSORS" and "expected F32" in msg
    # offsets that overlap
    hdr = json.loads(st[8:8 + n])
    names = [k for k in hdr if k != "__metadata__"]
    hdr[names[1]]["data_offsets"] = hdr[names[0]]["data_offsets"]
    h = json.dumps(hdr).encode()
    assert _status(t0hip, struct.pack("<Q", len(h)) + h + st[8 + n:], cj)[0] == "SAFETENSORS"


def test_refuses_bad_config(t0hip, checkpoint):
    st, cj, _, _ = checkpoint
    c = json.loads(cj)
    for mutate in (lambda d: d.pop("embed_dim"), lambda d: d.pop("dropout"),
                   lambda d: d.update(num_heads=-2), lambda d: d.update(patch_size=32.5),
                   lambda d: d.update(quantile_levels="0.5"), lambda d: d.update(scaler_use_arcsinh=1)):
        bad = dict(c)
        mutate(bad)
        assert _status(t0hip, st, json.dumps(bad))[0] == "CONFIG"
    assert _status(t0hip, st, "{not json")[0] == "CONFIG"
    # a config that does not match the tensors is caught by the model check on load
    wrong = dict(c, embed_dim=c["embed_dim"] * 2)
    g = t0hip.export_gguf_from_safetensors(st, json.dumps(wrong), 8)
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.inspect_gguf(g)
    assert e.value.status == "SHAPE"
