"""A small synthetic compressed-tensors checkpoint (two safetensors shards and
an index) for the loader tests."""
import json
import os

import numpy as np
import torch
from safetensors.torch import save_file

from pegainfer_amd import checkpoint, synth


def write_checkpoint(root, *, layer=3, experts=8, inter=128, hidden=256, seed=11,
                     single_file=False):
    """Returns {(expert, projection): (packed u8 [out, in/2], scale bits [out, in/32])}.
    Experts alternate between the two shards; each projection also carries a
    weight_shape tensor, and a neighbouring layer's expert 0 is present."""
    g = np.random.default_rng(seed)
    truth, shards = {}, ({}, {})
    for e in range(experts):
        for proj in checkpoint.PROJECTIONS:
            out_dim, in_dim = (hidden, inter) if proj == "down_proj" else (inter, hidden)
            packed, scale = synth.int4_checkpoint(g, 1, out_dim, in_dim)
            packed, scale = packed[0], scale[0]
            truth[(e, proj)] = (packed, scale)
            d = shards[e % 2]
            d[checkpoint.expert_tensor_name(layer, e, proj, "weight_packed")] = \
                torch.from_numpy(packed.copy()).view(torch.int32)
            d[checkpoint.expert_tensor_name(layer, e, proj, "weight_scale")] = \
                torch.from_numpy(scale.view(np.int16).copy()).view(torch.bfloat16)
            d[checkpoint.expert_tensor_name(layer, e, proj, "weight_packed").replace(
                "weight_packed", "weight_shape")] = torch.tensor([out_dim, in_dim], dtype=torch.int32)
    shards[0][checkpoint.expert_tensor_name(layer + 1, 0, "gate_proj", "weight_packed")] = \
        torch.zeros(4, dtype=torch.int32)
    if single_file:
        save_file({**shards[0], **shards[1]}, os.path.join(root, checkpoint.SINGLE_FILE))
        return truth
    names = ("model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors")
    weight_map = {}
    for fname, d in zip(names, shards):
        save_file(d, os.path.join(root, fname))
        weight_map.update({k: fname for k in d})
    with open(os.path.join(root, checkpoint.INDEX_FILE), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": weight_map}, f)
    return truth
