"""Write a decoder checkpoint in the Qwen3-ASR safetensors layout (tensor
names of the reference loader, qwen_asr_decoder.c:45-116) from a host model
object (pyoracle.SynthModel): BF16 matrices, norm vectors as F32 or BF16."""
import os

import numpy as np
import torch
from safetensors.torch import save_file


def layer_tensors(model, l, norm_bf16=False):
    wq, wk, wv, wo, gate, up, down, qn, kn, inn, pn = model.layer_args(l)
    p = f"thinker.model.layers.{l}."
    t = {}
    for name, w in (("self_attn.q_proj", wq), ("self_attn.k_proj", wk), ("self_attn.v_proj", wv),
                    ("self_attn.o_proj", wo), ("mlp.gate_proj", gate), ("mlp.up_proj", up),
                    ("mlp.down_proj", down)):
        t[p + name + ".weight"] = torch.from_numpy(np.ascontiguousarray(w).view(np.int16)).view(torch.bfloat16)
    for name, v in (("self_attn.q_norm", qn), ("self_attn.k_norm", kn), ("input_layernorm", inn),
                    ("post_attention_layernorm", pn)):
        v = torch.from_numpy(np.ascontiguousarray(v, np.float32))
        t[p + name + ".weight"] = v.to(torch.bfloat16) if norm_bf16 else v
    return t


def all_tensors(model, norm_bf16=False):
    t = {"thinker.model.embed_tokens.weight":
         torch.from_numpy(np.ascontiguousarray(model.emb).view(np.int16)).view(torch.bfloat16),
         "thinker.model.norm.weight": torch.from_numpy(np.ascontiguousarray(model.final_norm, np.float32))}
    for l in range(model.cfg.layers):
        t.update(layer_tensors(model, l, norm_bf16))
    return t


def write_checkpoint(model, path, shards=1, norm_bf16=False, extra=None):
    """model.safetensors, or `shards` files model-0000k-of-0000n.safetensors."""
    os.makedirs(path, exist_ok=True)
    t = all_tensors(model, norm_bf16)
    if extra:
        t.update(extra)
    names = sorted(t)
    if shards == 1:
        save_file(t, os.path.join(path, "model.safetensors"), metadata={"format": "pt"})
        return names
    per = (len(names) + shards - 1) // shards
    for k in range(shards):
        part = {n: t[n] for n in names[k * per:(k + 1) * per]}
        save_file(part, os.path.join(path, f"model-{k + 1:05d}-of-{shards:05d}.safetensors"),
                  metadata={"format": "pt"})
    return names


ENC_LAYER_NAMES = ("self_attn.q_proj.weight", "self_attn.q_proj.bias", "self_attn.k_proj.weight",
                   "self_attn.k_proj.bias", "self_attn.v_proj.weight", "self_attn.v_proj.bias",
                   "self_attn.out_proj.weight", "self_attn.out_proj.bias", "self_attn_layer_norm.weight",
                   "self_attn_layer_norm.bias", "fc1.weight", "fc1.bias", "fc2.weight", "fc2.bias",
                   "final_layer_norm.weight", "final_layer_norm.bias")
ENC_STEM_NAMES = ("conv2d1.weight", "conv2d1.bias", "conv2d2.weight", "conv2d2.bias", "conv2d3.weight",
                  "conv2d3.bias", "conv_out.weight", "ln_post.weight", "ln_post.bias", "proj1.weight",
                  "proj1.bias", "proj2.weight", "proj2.bias")
ENC_STEM_SHAPES = {"conv2d1.weight": (480, 1, 3, 3), "conv2d2.weight": (480, 480, 3, 3),
                   "conv2d3.weight": (480, 480, 3, 3)}


def enc_tensors(enc):
    """thinker.audio_tower.* of the encoder loader (qwen_asr_encoder.c:67-168)
    from a pyoracle.SynthEncoder: matrices as BF16 (the synthetic ones are
    bf16 values, so exact), vectors as F32."""
    def put(t, name, a):
        a = np.ascontiguousarray(a, np.float32)
        if a.ndim >= 2:
            bits = (a.view(np.uint32) >> 16).astype(np.uint16)
            t[name] = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
        else:
            t[name] = torch.from_numpy(a)

    t = {}
    for l, arrs in enumerate(enc.layers):
        for name, a in zip(ENC_LAYER_NAMES, arrs):
            put(t, f"thinker.audio_tower.layers.{l}.{name}", a)
    for name, a in zip(ENC_STEM_NAMES, enc.stem):
        if name in ENC_STEM_SHAPES:
            a = np.asarray(a).reshape(ENC_STEM_SHAPES[name])
        put(t, f"thinker.audio_tower.{name}", a)
    return t
