"""Local checkpoints (tsfm_attn.checkpoint): the safetensors reader and writer
(src/core/safetensors.zig:32-97) and the Chronos-Bolt config.json + model.safetensors layout
(src/chronos_bolt/config.zig:10-66, model.zig:101-160). CPU only.

The format is pinned against an independent implementation, the `safetensors` package: files it
writes are read here, and files written here load with it, value for value."""
import json

import numpy as np
import pytest

from tsfm_attn import checkpoint as ck


def _tensors(seed=0):
    rng = np.random.default_rng(seed)
    return {"a.weight": rng.standard_normal((3, 5)).astype(np.float32), "b": rng.standard_normal(7).astype(np.float32),
            "c.bias": np.array([1.0, -2.5, 3.140625, 0.0], np.float32)}


def test_round_trip_f32_in_place(tmp_path):
    t = _tensors()
    p = tmp_path / "m.safetensors"
    ck.write_safetensors(str(p), t)
    with ck.Weights(str(p)) as w:
        assert w.data_start % 8 == 0
        assert sorted(w.names()) == sorted(t)
        for k, v in t.items():
            got = w.get(k, v.size)
            assert got.dtype == np.float32 and np.array_equal(got, v.ravel())


def test_half_tensors_are_widened(tmp_path):
    """F16: the f16 value as f32. BF16: the 16 stored bits as the high half of an f32
    (safetensors.zig:81-91); the writer rounds to nearest even."""
    t = _tensors(1)
    for dt in ("F16", "BF16"):
        p = tmp_path / f"m_{dt}.safetensors"
        ck.write_safetensors(str(p), t, dt)
        with ck.Weights(str(p)) as w:
            for k, v in t.items():
                got = w.get(k, v.size)
                if dt == "F16":
                    want = v.ravel().astype(np.float16).astype(np.float32)
                else:
                    import torch

                    want = torch.from_numpy(v.ravel()).to(torch.bfloat16).float().numpy()
                assert np.array_equal(got, want), (dt, k)
    # exact bf16 values survive unchanged
    with ck.Weights(str(tmp_path / "m_BF16.safetensors")) as w:
        assert np.array_equal(w.get("c.bias", 4), t["c.bias"])


def test_errors_carry_the_reference_messages(tmp_path):
    p = tmp_path / "m.safetensors"
    ck.write_safetensors(str(p), _tensors())
    with ck.Weights(str(p)) as w:
        with pytest.raises(ck.SafetensorsError, match="missing tensor: nope"):
            w.get("nope", 1)
        with pytest.raises(ck.SafetensorsError, match="expected 8 elements, file has 7"):
            w.get("b", 8)
    hdr = json.dumps({"x": {"dtype": "I32", "shape": [2], "data_offsets": [0, 8]}}).encode()
    hdr += b" " * ((8 - (8 + len(hdr)) % 8) % 8)
    q = tmp_path / "i32.safetensors"
    q.write_bytes(len(hdr).to_bytes(8, "little") + hdr + b"\0" * 8)
    with ck.Weights(str(q)) as w:
        with pytest.raises(ck.SafetensorsError, match="unsupported dtype I32"):
            w.get("x", 2)
    (tmp_path / "short").write_bytes(b"\1\2")
    with pytest.raises(ck.SafetensorsError):
        ck.Weights(str(tmp_path / "short"))
    (tmp_path / "long_header").write_bytes((1 << 20).to_bytes(8, "little") + b"{}")
    with pytest.raises(ck.SafetensorsError):
        ck.Weights(str(tmp_path / "long_header"))


def test_interoperates_with_the_safetensors_package(tmp_path):
    st = pytest.importorskip("safetensors.numpy")
    t = _tensors(2)
    theirs = tmp_path / "theirs.safetensors"
    st.save_file(t, str(theirs))
    with ck.Weights(str(theirs)) as w:
        for k, v in t.items():
            assert np.array_equal(w.get(k, v.size), v.ravel())
    ours = tmp_path / "ours.safetensors"
    ck.write_safetensors(str(ours), t)
    back = st.load_file(str(ours))
    assert sorted(back) == sorted(t)
    for k, v in t.items():
        assert back[k].shape == v.shape and np.array_equal(back[k], v)


def _config(**kw):
    c = ck.bolt_config_dict(d_model=128, d_ff=256, num_heads=2, num_layers=1, num_decoder_layers=1,
                            context_length=2048, patch=16, prediction_length=16, quantiles=np.linspace(0.1, 0.9, 9))
    c.update(kw)
    return c


def test_bolt_config_defaults_and_validation():
    c = ck.parse_bolt_config(json.dumps(_config()))
    assert c["vocab"] == 2 and c["layer_norm_epsilon"] == 1e-6 and c["chronos_config"]["use_reg_token"]
    minimal = {k: v for k, v in _config().items() if k in ("d_model", "d_ff", "num_heads", "d_kv", "num_layers",
                                                           "num_decoder_layers", "chronos_config")}
    m = ck.parse_bolt_config(json.dumps(minimal))
    assert (m["relative_attention_num_buckets"], m["relative_attention_max_distance"]) == (32, 128)
    bad = [dict(dense_act_fn="gelu"), dict(relative_attention_num_buckets=31), dict(num_layers=0)]
    for b in bad:
        with pytest.raises(ValueError):
            ck.parse_bolt_config(json.dumps(_config(**b)))
    c2 = _config()
    c2["chronos_config"] = dict(c2["chronos_config"], input_patch_stride=8)
    with pytest.raises(ValueError, match="UnsupportedPatchStride"):
        ck.parse_bolt_config(json.dumps(c2))
    c3 = _config()
    c3["chronos_config"] = dict(c3["chronos_config"], use_reg_token=False)  # reg_token_id 1 >= vocab 1
    with pytest.raises(ValueError, match="token ids"):
        ck.parse_bolt_config(json.dumps(c3))


def test_bolt_checkpoint_round_trip(tmp_path):
    """A random-init checkpoint written and read back gives the same weights, and the file holds
    exactly the tensors the model reads, with the reference's names and element counts."""
    from tsfm_attn import workloads

    w = workloads.bolt_forward(B=2, n_patch=2, H=2, d_ff=256, n_layers=2, quantiles=9, horizon=16)
    a, m = w.arrays, w.meta
    weights = dict(reg=a["reg"], dec_start=a["dec_start"], rel_table=a["rel_table"], enc_final_norm=a["enc_final_norm"],
                   dec_final_norm=a["dec_final_norm"], enc=m["enc"], dec=m["dec"], ie=m["ie"], oe=m["oe"])
    cfg = _config(num_layers=2, num_decoder_layers=2)
    ck.write_bolt_checkpoint(str(tmp_path), cfg, weights)
    c, back = ck.read_bolt_weights(str(tmp_path))
    lay = ck.bolt_tensor_layout(c)
    with ck.Weights(str(tmp_path / "model.safetensors")) as f:
        assert sorted(f.names()) == sorted(lay)
        assert "encoder.block.1.layer.1.DenseReluDense.wo.weight" in lay
        assert "decoder.block.0.layer.1.EncDecAttention.k.weight" in lay
        assert "output_patch_embedding.residual_layer.bias" in lay
    for k in ("reg", "dec_start", "rel_table", "enc_final_norm", "dec_final_norm"):
        assert np.array_equal(back[k], weights[k]), k
    for part in ("enc", "dec"):
        for ly_b, ly_w in zip(back[part], weights[part]):
            for k in ly_w:
                assert np.array_equal(ly_b[k], ly_w[k]), (part, k)
    for part in ("ie", "oe"):
        for k in weights[part]:
            assert np.array_equal(back[part][k], weights[part][k]), (part, k)
