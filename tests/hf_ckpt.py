"""Test helper: small Hugging Face-style checkpoints (safetensors, BF16) of the synthetic
model, written with the Qwen2 tensor names the converter reads."""
from __future__ import annotations

import json
import struct

import numpy as np

from instantllm_amd import synth


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> BF16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def write_safetensors(path: str, tensors: dict[str, tuple[np.ndarray, str]]):
    """tensors: name -> (array already in the stored dtype, safetensors dtype name)."""
    header, blobs, off = {}, [], 0
    for name, (a, dt) in tensors.items():
        b = np.ascontiguousarray(a).tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def checkpoint_tensors(seed: int, shape: synth.ModelShape) -> dict[str, np.ndarray]:
    """The synthetic model's float tensors under Qwen2 names, rounded to BF16 (float32)."""
    t = {"model.embed_tokens.weight": synth.float_embed(seed, shape), "model.norm.weight": synth.float_norm(seed, shape)}
    names = {"ln1": "input_layernorm.weight", "ln2": "post_attention_layernorm.weight",
             "wq": "self_attn.q_proj.weight", "bq": "self_attn.q_proj.bias", "wk": "self_attn.k_proj.weight",
             "bk": "self_attn.k_proj.bias", "wv": "self_attn.v_proj.weight", "bv": "self_attn.v_proj.bias",
             "wo": "self_attn.o_proj.weight", "wg": "mlp.gate_proj.weight", "wu": "mlp.up_proj.weight",
             "wd": "mlp.down_proj.weight"}
    for l in range(shape.layers):
        for k, v in synth.float_layer(seed, l, shape).items():
            t[f"model.layers.{l}.{names[k]}"] = v
    return {k: from_bf16_bits(to_bf16_bits(v)) for k, v in t.items()}


def write_checkpoint(directory: str, tensors: dict[str, np.ndarray], shards: int = 1):
    """Write `tensors` (float32 holding BF16 values) as BF16 safetensors: one
    model.safetensors, or `shards` files plus model.safetensors.index.json."""
    items = list(tensors.items())
    if shards == 1:
        write_safetensors(f"{directory}/model.safetensors", {k: (to_bf16_bits(v), "BF16") for k, v in items})
        return
    wm = {}
    per = (len(items) + shards - 1) // shards
    for s in range(shards):
        fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        part = items[s * per:(s + 1) * per]
        write_safetensors(f"{directory}/{fn}", {k: (to_bf16_bits(v), "BF16") for k, v in part})
        wm.update({k: fn for k, _ in part})
    with open(f"{directory}/model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
