"""Writes the tiny C1 model as a Qwen3.5-style checkpoint directory:
config.json plus safetensors files holding the CPU oracle's synthetic
weights under the reference's tensor names (models/qwen3_weights.cc:196-380:
model.language_model.layers.{i}.*, mtp.*, lm_head.weight).  With fp8=True the
QuantizedWeight Linears are stored as F8_E4M3 codes with a 128 x 128
weight_scale_inv grid -- the codes and scales of the oracle's own FP8 model
(its synthetic scales, its encoder) -- so that a loaded checkpoint must
reproduce the oracle's bf16 or FP8 model bit for bit.  The directory also
gets the small byte-level tokenizer of tests/tok.py.  Test helper only."""
import json
from pathlib import Path

import numpy as np
import torch
from safetensors.torch import save_file

import tok
from _hai import orc

# layer tensor kinds (slot * 64 + kind), as the engine and the oracle number them
LAYER_NAMES = {
    0: "input_layernorm.weight", 1: "post_attention_layernorm.weight", 2: "linear_attn.in_proj_qkv.weight",
    3: "linear_attn.in_proj_z.weight", 4: "linear_attn.in_proj_a.weight", 5: "linear_attn.in_proj_b.weight",
    6: "linear_attn.conv1d.weight", 7: "linear_attn.A_log", 8: "linear_attn.dt_bias", 9: "linear_attn.norm.weight",
    10: "linear_attn.out_proj.weight", 11: "self_attn.q_proj.weight", 12: "self_attn.k_proj.weight",
    13: "self_attn.v_proj.weight", 14: "self_attn.o_proj.weight", 15: "self_attn.q_norm.weight",
    16: "self_attn.k_norm.weight", 17: "mlp.gate_proj.weight", 18: "mlp.up_proj.weight", 19: "mlp.down_proj.weight",
}
QUANTIZED = {2, 3, 10, 11, 12, 13, 14, 17, 18, 19}  # the reference's QuantizedWeight Linears


def tensor_list(c):
    """(id, name, shape) of every weight of config c."""
    H, F, V = c["hidden"], c["ffn"], c["vocab"]
    qw, kvw, D = c["num_q_heads"] * c["head_dim"], c["num_kv_heads"] * c["head_dim"], c["head_dim"]
    kw, vw = c["lin_qk_heads"] * c["lin_k_dim"], c["lin_v_heads"] * c["lin_v_dim"]
    C, nv, dv, Kc = 2 * kw + vw, c["lin_v_heads"], c["lin_v_dim"], c["conv_kernel"]
    out = [(0, "model.language_model.embed_tokens.weight", (V, H)), (1, "model.language_model.norm.weight", (H,)),
           (2, "lm_head.weight", (V, H)), (64, "mtp.fc.weight", (H, 2 * H)), (65, "mtp.norm.weight", (H,)),
           (66, "mtp.pre_fc_norm_embedding.weight", (H,)), (67, "mtp.pre_fc_norm_hidden.weight", (H,))]
    attn_shapes = {0: (H,), 1: (H,), 11: (2 * qw, H), 12: (kvw, H), 13: (kvw, H), 14: (H, qw), 15: (D,), 16: (D,),
                   17: (F, H), 18: (F, H), 19: (H, F)}
    lin_shapes = {0: (H,), 1: (H,), 2: (C, H), 3: (vw, H), 4: (nv, H), 5: (nv, H), 6: (C, 1, Kc), 7: (nv,), 8: (nv,),
                  9: (dv,), 10: (H, vw), 17: (F, H), 18: (F, H), 19: (H, F)}
    layers = [(2 + i, f"model.language_model.layers.{i}.", (i + 1) % c["full_attention_interval"] == 0)
              for i in range(c["num_layers"])] + [(1024, "mtp.layers.0.", True)]
    for slot, prefix, attn in layers:
        for kind, shape in (attn_shapes if attn else lin_shapes).items():
            out.append((slot * 64 + kind, prefix + LAYER_NAMES[kind], shape))
    return out


def config_json(c, eos=None, **overrides):
    text = {
        "hidden_size": c["hidden"], "num_hidden_layers": c["num_layers"], "num_attention_heads": c["num_q_heads"],
        "num_key_value_heads": c["num_kv_heads"], "head_dim": c["head_dim"], "intermediate_size": c["ffn"],
        "vocab_size": c["vocab"], "max_position_embeddings": 4096, "rms_norm_eps": c["rms_eps"],
        "linear_num_key_heads": c["lin_qk_heads"], "linear_num_value_heads": c["lin_v_heads"],
        "linear_key_head_dim": c["lin_k_dim"], "linear_value_head_dim": c["lin_v_dim"],
        "linear_conv_kernel_dim": c["conv_kernel"], "full_attention_interval": c["full_attention_interval"],
        "layer_types": ["full_attention" if (i + 1) % c["full_attention_interval"] == 0 else "linear_attention"
                        for i in range(c["num_layers"])],
        "rope_parameters": {"rope_theta": c["rope_theta"], "partial_rotary_factor": c["rope_dim"] / c["head_dim"]},
        "mtp_num_hidden_layers": c["mtp_layers"], "attn_output_gate": True,
    }
    if eos is not None:
        text["eos_token_id"] = eos
    text.update(overrides)
    return {"architectures": ["Qwen3_5ForConditionalGeneration"], "model_type": "qwen3_5", "text_config": text,
            "tie_word_embeddings": False}


def write_tiny_checkpoint(path, fp8=False, shards=1, eos=None, scale_dtype=torch.float32, generation_eos=None):
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    c = orc.TINY
    m = orc.Model(c, seed=0)
    tensors = {}
    try:
        for tid, name, shape in tensor_list(c):
            w = m.tensor(tid).astype(np.float32).reshape(shape)
            if fp8 and tid % 64 in QUANTIZED and tid >= 128:
                rows, cols = shape
                nbr, nbc = (rows + 127) // 128, (cols + 127) // 128
                s = orc.fp8_synthetic_scales(0, tid, nbr * nbc).reshape(nbr, nbc)
                expand = np.repeat(np.repeat(s, 128, 0), 128, 1)[:rows, :cols]
                q = orc.fp8_encode(w / expand)
                tensors[name] = torch.from_numpy(np.ascontiguousarray(q)).view(torch.float8_e4m3fn)
                tensors[name[:-len(".weight")] + ".weight_scale_inv"] = torch.from_numpy(s).to(scale_dtype)
            else:
                tensors[name] = torch.from_numpy(np.ascontiguousarray(w)).to(torch.bfloat16)
    finally:
        m.close()
    (path / "config.json").write_text(json.dumps(config_json(c, eos)))
    names = sorted(tensors)
    if shards == 1:
        save_file(tensors, str(path / "model.safetensors"))
    else:
        weight_map = {}
        for k in range(shards):
            part = names[k::shards]
            fname = f"model-{k + 1:05d}-of-{shards:05d}.safetensors"
            save_file({n: tensors[n] for n in part}, str(path / fname))
            weight_map.update({n: fname for n in part})
        (path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    # the tokenizer (tests/tok.py: ids below the tiny vocabulary) and, when
    # given, generation_config.json's stop ids
    tok.write_tokenizer(path, generation=None if generation_eos is None else {"eos_token_id": generation_eos})
    return path
