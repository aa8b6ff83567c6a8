"""GGUF container, config recovery, export policy and the failure paths a host
can force with corrupted bytes (CPU; no GPU needed: t0h_gguf_inspect parses and
validates exactly what t0h_model_load_gguf does before touching a device).

Reference: crates/t0-core/src/gguf.rs:228-482, weights.rs:32-37, 69-112, 187-227,
config.rs:45-56, model.rs:84-147."""
import struct

import numpy as np
import pytest

import gguf_py as G
from util import TINY


def tiny_tensors(oracle, E=128, H=256, heads=2, ps=32, nq=3, layers=3, ty=1, drop=None):
    """Every tensor T0Model::load needs, F16 (or `ty` for the big matmuls)."""
    rng = np.random.default_rng(0)
    hd = E // heads
    spec = [("patch_encoder.projection.mlp.hidden_layer.weight", [E, 3 * ps]),
            ("patch_encoder.projection.mlp.hidden_layer.bias", [E]),
            ("patch_encoder.projection.mlp.output_layer.weight", [E, E]),
            ("patch_encoder.projection.mlp.output_layer.bias", [E]),
            ("patch_encoder.projection.residual_layer.weight", [E, 3 * ps]),
            ("patch_encoder.projection.residual_layer.bias", [E]),
            ("patch_encoder.type_embeddings.weight", [3, E]),
            ("transformer.out_norm.scale", [E]),
            ("decoder.mlp.hidden_layer.weight", [E, E]), ("decoder.mlp.hidden_layer.bias", [E]),
            ("decoder.mlp.output_layer.weight", [ps * nq, E]), ("decoder.mlp.output_layer.bias", [ps * nq]),
            ("decoder.residual_layer.weight", [ps * nq, E]), ("decoder.residual_layer.bias", [ps * nq])]
    for i in range(layers):
        p = f"transformer.layers.{i}"
        spec += [(f"{p}.attention_block.norm.scale", [E]),
                 (f"{p}.attention_block.attention.wQKV.weight", [3 * E, E]),
                 (f"{p}.attention_block.attention.wQKV.bias", [3 * E]),
                 (f"{p}.attention_block.attention.wO.weight", [E, E]),
                 (f"{p}.attention_block.attention.wO.bias", [E]),
                 (f"{p}.attention_block.attention.q_norm.scale", [hd]),
                 (f"{p}.attention_block.attention.k_norm.scale", [hd]),
                 (f"{p}.norm.scale", [E]), (f"{p}.mlp.0.weight", [2 * H, E]), (f"{p}.mlp.0.bias", [2 * H]),
                 (f"{p}.mlp.2.weight", [E, H]), (f"{p}.mlp.2.bias", [E])]
    out = []
    for name, shape in spec:
        if name == drop:
            continue
        x = (0.02 * rng.standard_normal(int(np.prod(shape)))).astype(np.float32)
        big = len(shape) == 2 and any(s in name for s in (".wQKV.weight", ".wO.weight", ".mlp.0.weight", ".mlp.2.weight"))
        t = ty if big else 1
        out.append((name, shape, t, oracle.quantize(t, x).tobytes()))
    return out


def status_of(t0hip, b):
    try:
        t0hip.inspect_gguf(b)
        return "OK"
    except t0hip.T0HipError as e:
        return e.status


def oracle_status(oracle, b):
    try:
        oracle.Model(b)
        return 0
    except oracle.OracleError as e:
        return e.code


def test_reference_round_trip(oracle):
    """gguf.rs:435-481: shape, type and metadata survive a round trip (here through the
    oracle's reader of an independently encoded file)."""
    a = (np.sin(np.arange(64, dtype=np.float32) * np.float32(0.37)) * 3).astype(np.float32)
    b = (np.sin(np.arange(320, dtype=np.float32) * np.float32(0.37)) * 3).astype(np.float32)
    meta = G.t0_meta(embed=128, heads=2, levels=(0.1, 0.5, 0.9)) + [("t0.scaler_eps_mode", G.STRING, "variance_offset")]
    tensors = tiny_tensors(oracle) + [("norm.scale", [64], 0, a.tobytes()),
                                      ("layer.weight", [10, 32], 8, oracle.quantize(8, b).tobytes())]
    m = oracle.Model(G.build(meta, tensors))
    assert m.cfg.embed_dim == 128 and m.n_q == 3
    np.testing.assert_array_equal(m.tensor("norm.scale"), a)
    lw = m.tensor("layer.weight")
    assert lw.shape == (10, 32)
    assert np.max(np.abs(lw.ravel() - b)) < 0.03


def test_product_and_oracle_accept_the_same_file(oracle, t0hip):
    b = G.build(G.t0_meta(), tiny_tensors(oracle, ty=8))
    cfg, n = t0hip.inspect_gguf(b)
    assert (cfg.embed_dim, cfg.num_layers, cfg.num_heads, cfg.n_quantiles) == (128, 3, 2, 3)
    assert n == len(tiny_tensors(oracle))
    assert oracle_status(oracle, b) == 0


def test_config_defaults_and_modes(oracle, t0hip):
    """weights.rs:76-111: optional keys fall back to dropout 0, arcsinh true, eps 0.1,
    variance_offset; any eps mode other than "std_clamp" is variance_offset."""
    t = tiny_tensors(oracle)
    cfg, _ = t0hip.inspect_gguf(G.build(G.t0_meta(), t))
    assert cfg.dropout == 0.0 and cfg.scaler_use_arcsinh == 1 and cfg.scaler_eps == np.float32(0.1)
    assert cfg.scaler_variance_offset == 1
    extra = [("t0.scaler_eps_mode", G.STRING, "std_clamp"), ("t0.scaler_eps", G.F32, 0.01),
             ("t0.scaler_use_arcsinh", G.BOOL, False), ("t0.dropout", G.F32, 0.25)]
    cfg, _ = t0hip.inspect_gguf(G.build(G.t0_meta(extra=extra), t))
    assert cfg.scaler_variance_offset == 0 and cfg.scaler_use_arcsinh == 0
    assert cfg.scaler_eps == np.float32(0.01) and cfg.dropout == 0.25
    cfg, _ = t0hip.inspect_gguf(G.build(G.t0_meta(extra=[("t0.scaler_eps_mode", G.STRING, "anything")]), t))
    assert cfg.scaler_variance_offset == 1
    # an optional key of the wrong type falls back to its default (the reference's `_ => default`)
    cfg, _ = t0hip.inspect_gguf(G.build(G.t0_meta(extra=[("t0.scaler_eps", G.U32, 5)]), t))
    assert cfg.scaler_eps == np.float32(0.1)


def test_layer_types(oracle, t0hip):
    """config.rs:45-56: (n-1) TIME then GROUP, repeated num_layers/n times (truncating)."""
    for layers, gen, want in ((3, 3, 3), (6, 3, 6), (4, 3, 3), (5, 0, 5)):
        t = tiny_tensors(oracle, layers=layers)
        b = G.build(G.t0_meta(layers=layers, gen=gen), t)
        cfg, _ = t0hip.inspect_gguf(b)
        assert oracle.Model(b).cfg.num_layers == want


CASES = {
    "bad magic": (lambda o: G.build(G.t0_meta(), tiny_tensors(o), magic=b"GGUX"), "GGUF_MAGIC", -2),
    "version 2": (lambda o: G.build(G.t0_meta(), tiny_tensors(o), version=2), "GGUF_VERSION", -3),
    "tensor type 7": (lambda o: G.build(G.t0_meta(), tiny_tensors(o)[:1] + [("x", [32], 7, b"\0" * 64)]),
                      "GGUF_TENSOR_TYPE", -4),
    "meta type i32": (lambda o: G.build(G.t0_meta(), tiny_tensors(o), raw_meta=[("k", struct.pack("<Ii", 5, 1))]),
                      "GGUF_META_TYPE", -5),
    "u32 array": (lambda o: G.build(G.t0_meta(), tiny_tensors(o), raw_meta=[("k", struct.pack("<IIQI", 9, 4, 1, 7))]),
                  "GGUF_META_TYPE", -5),
    "offset past blob": (lambda o: G.build(G.t0_meta(), tiny_tensors(o)[:2],
                                           offsets=[0, 1 << 30]), "GGUF_BOUNDS", -6),
    "truncated": (lambda o: G.build(G.t0_meta(), tiny_tensors(o))[:-100], "GGUF_BOUNDS", -6),
    "truncated header": (lambda o: G.build(G.t0_meta(), tiny_tensors(o))[:30], "GGUF_BOUNDS", -6),
    "missing tensor": (lambda o: G.build(G.t0_meta(), tiny_tensors(o, drop="transformer.layers.1.mlp.2.bias")),
                       "MISSING_TENSOR", -7),
    "missing key": (lambda o: G.build(G.t0_meta()[1:], tiny_tensors(o)), "METADATA", -8),
    "wrong-typed key": (lambda o: G.build([("t0.embed_dim", G.F32, 128.0)] + G.t0_meta()[1:], tiny_tensors(o)),
                        "METADATA", -8),
    "missing levels": (lambda o: G.build(G.t0_meta()[:-1], tiny_tensors(o)), "METADATA", -8),
    "bad utf-8": (lambda o: G.build(G.t0_meta(), tiny_tensors(o), raw_meta=[(b"\xff\xfe", G.meta_value(G.U32, 1))]),
                  "METADATA", -8),
    "q8 count % 32": (lambda o: G.build(G.t0_meta(), tiny_tensors(o) + [("odd", [33], 8, b"\0" * 68)]), "SHAPE", -13),
    "shape mismatch": (lambda o: G.build(G.t0_meta(embed=256), tiny_tensors(o)), "SHAPE", -13),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_failure_paths(oracle, t0hip, case):
    make, status, code = CASES[case]
    b = make(oracle)
    assert status_of(t0hip, b) == status
    assert oracle_status(oracle, b) == code


def test_export_matches_oracle_byte_for_byte(oracle, t0hip):
    """Weights::export_gguf (weights.rs:187-227): sorted names, the four big matmuls quantized,
    everything else F16, 32-byte aligned blob offsets.  Product and oracle writers agree."""
    cfg = t0hip.make_config(**TINY)
    f32 = t0hip.synth_model_gguf(cfg, quant=0, seed=3)
    om = oracle.Model(f32)
    for q in (1, 8, 2, 0):
        a = om.export_gguf(q)
        assert a == t0hip.export_gguf(f32, q)
        assert a == t0hip.synth_model_gguf(cfg, quant=q, seed=3)
        m = oracle.Model(a)
        w = m.tensor("transformer.layers.0.mlp.0.weight")
        assert w.shape == (2 * cfg.mlp_hidden_dim, cfg.embed_dim)


def test_export_policy_types(oracle, t0hip):
    """Only rank-2 tensors named like the four big matmuls take the requested type."""
    g = t0hip.synth_model_gguf(t0hip.make_config(**TINY), quant=2, seed=1)
    blob = np.frombuffer(g, np.uint8)
    # parse tensor infos with the test encoder's layout
    pos = 4 + 4 + 16
    n_t, n_m = struct.unpack_from("<QQ", g, 8)

    def rstr(p):
        n = struct.unpack_from("<Q", g, p)[0]
        return g[p + 8:p + 8 + n].decode(), p + 8 + n

    for _ in range(n_m):
        _, pos = rstr(pos)
        ty = struct.unpack_from("<I", g, pos)[0]
        pos += 4
        if ty == 4 or ty == 6:
            pos += 4
        elif ty == 7:
            pos += 1
        elif ty == 8:
            _, pos = rstr(pos)
        elif ty == 9:
            n = struct.unpack_from("<Q", g, pos + 4)[0]
            pos += 12 + 4 * n
    names = []
    for _ in range(n_t):
        name, pos = rstr(pos)
        nd = struct.unpack_from("<I", g, pos)[0]
        pos += 4 + 8 * nd
        ty, off = struct.unpack_from("<IQ", g, pos)
        pos += 12
        big = any(s in name for s in (".attention.wQKV.weight", ".attention.wO.weight", ".mlp.0.weight", ".mlp.2.weight"))
        assert ty == (2 if big else 1), name
        assert off % 32 == 0
        names.append(name)
    assert names == sorted(names)
    assert blob.size > 0
