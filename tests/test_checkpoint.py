"""Checkpoint files on the CPU (no device): config.json read by the rules of
the reference's Qwen3Config::load_json (models/qwen3_config.cc:12-206),
safetensors headers validated as its SafeTensorLoader does
(io/safetensor_loader.cc:73-404: header length, dtypes, dims, offsets,
byte counts, sharded indexes), and the Linear format detected from the
checkpoint (dense BF16, or F8_E4M3 with weight_scale_inv; a mixture is
refused).  Status numbers are the reference's StatusCode values."""
import json
import struct

import pytest
import torch
from safetensors.torch import save_file

import ckpt
from _hai import orc

FILE_NOT_FOUND, INVALID_MODEL, UNSUPPORTED_DTYPE, NOT_IMPLEMENTED = 7, 8, 6, 3


@pytest.fixture(scope="module")
def E():
    from hybridai_amd import engine
    return engine


@pytest.fixture(scope="module")
def tiny_dir(tmp_path_factory):
    return ckpt.write_tiny_checkpoint(tmp_path_factory.mktemp("tiny"), eos=[7, 11])


def write_config(d, **overrides):
    d.mkdir(parents=True, exist_ok=True)
    (d / "config.json").write_text(json.dumps(ckpt.config_json(orc.TINY, **overrides)))
    return d


def code_of(E, d, weight_format=False):
    try:
        E.model_config_load(d, weight_format)
    except E.CheckpointError as e:
        return e.code
    return 0


def test_config_and_format_of_a_tiny_checkpoint(E, tiny_dir, tmp_path):
    cfg, eos, fmt = E.model_config_load(tiny_dir)
    for k, v in orc.TINY.items():
        assert cfg[k] == pytest.approx(v, rel=1e-6), k
    assert eos == [7, 11] and fmt == E.WEIGHTS_BF16
    fp8_dir = ckpt.write_tiny_checkpoint(tmp_path / "fp8", fp8=True, shards=3)
    assert E.model_config_load(fp8_dir)[2] == E.WEIGHTS_FP8_BLOCK128


def test_config_rules(E, tmp_path):
    # head_dim absent: hidden / heads; rope_theta and the rotary fraction from rope_parameters
    d = write_config(tmp_path / "a", head_dim=None)
    raw = json.loads((d / "config.json").read_text())
    del raw["text_config"]["head_dim"]
    raw["text_config"]["rope_parameters"] = {"rope_theta": 5e6, "partial_rotary_factor": 0.5}
    (d / "config.json").write_text(json.dumps(raw))
    cfg, _, _ = E.model_config_load(d, False)
    assert cfg["head_dim"] == 64 and cfg["rope_dim"] == 32 and cfg["rope_theta"] == 5e6
    # text_config fields win over the root's; root fields fill the rest
    raw = ckpt.config_json(orc.TINY)
    raw["hidden_size"] = 999
    raw["eos_token_id"] = 5
    (d / "config.json").write_text(json.dumps(raw))
    cfg, eos, _ = E.model_config_load(d, False)
    assert cfg["hidden"] == 256 and eos == [5]
    # defaults of the reference (the 27B shape) for an empty config
    (d / "config.json").write_text("{}")
    cfg, eos, _ = E.model_config_load(d, False)
    assert (cfg["hidden"], cfg["num_layers"], cfg["vocab"], cfg["rope_dim"], cfg["mtp_layers"]) == \
           (5120, 64, 248320, 64, 0) and eos == []


@pytest.mark.parametrize("change,code", [
    (dict(layer_types=["full_attention"] * 4), INVALID_MODEL),                 # conflicts with the interval
    (dict(layer_types=["linear_attention"] * 3 + ["sliding"]), INVALID_MODEL),  # unknown type
    (dict(layer_types=["linear_attention"] * 3), INVALID_MODEL),               # wrong count
    (dict(attn_output_gate=False), INVALID_MODEL),
    (dict(mamba_ssm_dtype="bfloat16"), INVALID_MODEL),
    (dict(eos_token_id="2"), INVALID_MODEL),
    (dict(eos_token_id=[1, "x"]), INVALID_MODEL),
    (dict(num_key_value_heads=3), INVALID_MODEL),                              # heads % kv_heads
    (dict(mtp_num_hidden_layers=-1), INVALID_MODEL),
])
def test_config_errors(E, tmp_path, change, code):
    write_config(tmp_path, **change)
    assert code_of(E, tmp_path) == code


def test_config_missing_and_malformed(E, tmp_path):
    assert code_of(E, tmp_path / "none") == FILE_NOT_FOUND
    tmp_path.joinpath("config.json").write_text('{"text_config": {"hidden_size": 256,}')
    assert code_of(E, tmp_path) == INVALID_MODEL


def raw_safetensors(path, header, data=b""):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)


@pytest.mark.parametrize("case,code", [
    ("header_past_end", INVALID_MODEL), ("offsets_past_data", INVALID_MODEL), ("bytes_not_shape", INVALID_MODEL),
    ("negative_dim", INVALID_MODEL), ("unknown_dtype", UNSUPPORTED_DTYPE), ("not_json", INVALID_MODEL),
    ("no_offsets", INVALID_MODEL)])
def test_safetensors_header_validation(E, tmp_path, case, code):
    write_config(tmp_path)
    f = tmp_path / "model.safetensors"
    if case == "header_past_end":
        f.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    elif case == "offsets_past_data":
        raw_safetensors(f, {"a": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [0, 8]}}, b"\0" * 4)
    elif case == "bytes_not_shape":
        raw_safetensors(f, {"a": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 8]}}, b"\0" * 8)
    elif case == "negative_dim":
        raw_safetensors(f, {"a": {"dtype": "BF16", "shape": [-2, 2], "data_offsets": [0, 8]}}, b"\0" * 8)
    elif case == "unknown_dtype":
        raw_safetensors(f, {"a": {"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}}, b"\0" * 8)
    elif case == "not_json":
        h = b"{not json"
        f.write_bytes(struct.pack("<Q", len(h)) + h)
    elif case == "no_offsets":
        raw_safetensors(f, {"a": {"dtype": "BF16", "shape": [2, 2]}}, b"\0" * 8)
    assert code_of(E, tmp_path, True) == code


def test_sharded_index_and_missing_tensors(E, tiny_dir, tmp_path):
    # a tensor listed in the index but absent from its shard
    d = ckpt.write_tiny_checkpoint(tmp_path / "sharded", shards=2)
    idx = json.loads((d / "model.safetensors.index.json").read_text())
    shard = idx["weight_map"]["lm_head.weight"]
    idx["weight_map"]["ghost.weight"] = shard
    (d / "model.safetensors.index.json").write_text(json.dumps(idx))
    assert code_of(E, d, True) == INVALID_MODEL
    # neither an index nor model.safetensors
    write_config(tmp_path / "empty")
    assert code_of(E, tmp_path / "empty", True) == FILE_NOT_FOUND
    # a required Linear missing
    from safetensors.torch import load_file
    t = load_file(str(tiny_dir / "model.safetensors"))
    del t["model.language_model.layers.1.mlp.up_proj.weight"]
    write_config(tmp_path / "missing")
    save_file(t, str(tmp_path / "missing" / "model.safetensors"))
    assert code_of(E, tmp_path / "missing", True) == INVALID_MODEL


def test_mixed_dense_and_fp8_linears_are_refused(E, tiny_dir, tmp_path):
    from safetensors.torch import load_file
    t = load_file(str(tiny_dir / "model.safetensors"))
    name = "model.language_model.layers.0.mlp.down_proj.weight"
    w = t[name].float().numpy()
    t[name] = torch.from_numpy(orc.fp8_encode(w / 0.01)).view(torch.float8_e4m3fn)
    t[name[:-7] + ".weight_scale_inv"] = torch.full(((w.shape[0] + 127) // 128, (w.shape[1] + 127) // 128), 0.01)
    write_config(tmp_path)
    save_file(t, str(tmp_path / "model.safetensors"))
    assert code_of(E, tmp_path, True) == NOT_IMPLEMENTED
    # an FP8 Linear without its scale grid is not a QuantizedWeight
    del t[name[:-7] + ".weight_scale_inv"]
    save_file(t, str(tmp_path / "model.safetensors"))
    assert code_of(E, tmp_path, True) == UNSUPPORTED_DTYPE


def test_dense_tensors_must_hold_bf16_values(E, tiny_dir, tmp_path):
    """The non-Linear tensors are stored as BF16, the dtype the reference's
    GPU ops take them in (delta_net.cc:477-478): an F16 A_log, or an F32
    A_log whose values are not bf16 numbers, is refused before any device
    work with UNSUPPORTED_DTYPE and the tensor's name; F32 holding bf16
    values loads as before."""
    from safetensors.torch import load_file
    t = load_file(str(tiny_dir / "model.safetensors"))
    name = "model.language_model.layers.0.linear_attn.A_log"
    base = t[name].float()
    cases = (("f16", base.to(torch.float16), UNSUPPORTED_DTYPE, "is F16"),
             ("f32_off", (base.double() * (1 + 2.0 ** -10) + 2.0 ** -20).float(), UNSUPPORTED_DTYPE,
              "not bf16 numbers"),
             ("f32_exact", base, 0, ""))
    for tag, value, want, text in cases:
        d = write_config(tmp_path / tag)
        save_file(dict(t, **{name: value.contiguous()}), str(d / "model.safetensors"))
        assert code_of(E, d, True) == want, tag
        if want:
            with pytest.raises(E.CheckpointError, match=text) as ei:
                E.model_config_load(d, True)
            assert name in str(ei.value)


def with_metadata_text(src, dst, text_json_literal):
    """Copy of a safetensors file whose header gains
    "__metadata__": {"note": <literal>} (the literal written as given)."""
    raw = src.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    header, data = raw[8:8 + n], raw[8 + n:]
    assert header.startswith(b"{")
    header = b'{"__metadata__": {"note": ' + text_json_literal + b"}, " + header[1:]
    dst.write_bytes(struct.pack("<Q", len(header)) + header + data)


def test_unicode_and_escapes_in_json(E, tiny_dir, tmp_path):
    """The header reader decodes escapes and surrogate pairs and refuses an
    unpaired surrogate: the same complete checkpoint loads with the first
    note and is refused with the second."""
    write_config(tmp_path / "good")
    with_metadata_text(tiny_dir / "model.safetensors", tmp_path / "good" / "model.safetensors",
                       b'"caf\\u00e9 \\ud83d\\ude00 \\"q\\" \\\\ \\/"')
    assert code_of(E, tmp_path / "good", True) == 0
    write_config(tmp_path / "bad")
    with_metadata_text(tiny_dir / "model.safetensors", tmp_path / "bad" / "model.safetensors", b'"\\ud83d"')
    assert code_of(E, tmp_path / "bad", True) == INVALID_MODEL
