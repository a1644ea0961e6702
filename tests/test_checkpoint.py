"""Checkpoint loader (host side): names, index parsing, expert-major reads,
dtype/shape checks, and the I32 word <-> byte layout.  The GPU repack of what
it reads is in test_gpu_repack.py."""
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from ckpt_helpers import write_checkpoint
from pegainfer_amd import checkpoint


def test_expert_tensor_names_follow_the_reference():
    # manifest.rs:698-721 with the layer prefix of manifest.rs:711-719; a name the
    # reference's tests use (weights/tests.rs:147)
    assert checkpoint.expert_tensor_name(1, 143, "gate_proj", "weight_packed") == \
        "language_model.model.layers.1.mlp.experts.143.gate_proj.weight_packed"
    assert checkpoint.expert_tensor_name(1, 191, "down_proj", "weight_scale") == \
        "language_model.model.layers.1.mlp.experts.191.down_proj.weight_scale"
    with pytest.raises(ValueError):
        checkpoint.expert_tensor_name(1, 0, "down_proj", "weight_shape")
    assert checkpoint.rank_expert_range(3, 48, 384) == range(144, 192)
    with pytest.raises(ValueError):
        checkpoint.rank_expert_range(8, 48, 384)


def test_weight_shape_is_never_read():
    names = [n for pair in checkpoint.projection_tensor_names(1, range(144, 192), "down_proj")
             for n in pair]
    assert len(names) == 96 and not any(n.endswith("weight_shape") for n in names)


@pytest.mark.parametrize("single_file", [False, True])
def test_read_projection_is_expert_major_and_exact(tmp_path, single_file):
    truth = write_checkpoint(str(tmp_path), single_file=single_file)
    index = checkpoint.CheckpointIndex.from_model_dir(str(tmp_path))
    experts = checkpoint.rank_expert_range(1, 4, 8)  # experts 4..7, both shards
    for proj in checkpoint.PROJECTIONS:
        out_dim, in_dim = (256, 128) if proj == "down_proj" else (128, 256)
        packed, scale = checkpoint.read_projection(index, 3, experts, proj, out_dim, in_dim)
        assert packed.dtype == torch.int32 and packed.shape == (4, out_dim, in_dim // 8)
        for i, e in enumerate(experts):
            p, s = truth[(e, proj)]
            # the I32 words' little-endian bytes are the byte-per-column-pair layout
            assert np.array_equal(packed[i].view(torch.uint8).numpy(), p)
            assert np.array_equal(scale[i].view(torch.int16).numpy().view(np.uint16), s)


def test_nibble_order_of_an_i32_word():
    # element k of a word sits at bits [4k, 4k+4) (experts.rs:1606-1628): byte j
    # holds elements 2j (low nibble) and 2j+1 (high nibble)
    word = sum((k + 1) << (4 * k) for k in range(7)) | (8 << 28)  # elements 1..7, 8
    b = np.array([word], dtype=np.uint32).view(np.uint8)
    assert [int(x) & 15 for x in b] == [1, 3, 5, 7] and [int(x) >> 4 for x in b] == [2, 4, 6, 8]


def test_loader_rejects_bad_checkpoints(tmp_path):
    write_checkpoint(str(tmp_path))
    index = checkpoint.CheckpointIndex.from_model_dir(str(tmp_path))
    with pytest.raises(KeyError, match="experts.8.gate_proj.weight_packed"):
        checkpoint.read_projection(index, 3, range(6, 9), "gate_proj", 128, 256)
    with pytest.raises(ValueError, match="shape"):
        checkpoint.read_projection(index, 3, range(0, 2), "gate_proj", 64, 256)
    # a tensor with the right name and the wrong dtype
    bad = tmp_path / "bad"
    bad.mkdir()
    name = checkpoint.expert_tensor_name(0, 0, "up_proj", "weight_packed")
    sname = checkpoint.expert_tensor_name(0, 0, "up_proj", "weight_scale")
    save_file({name: torch.zeros(128, 32, dtype=torch.int16),
               sname: torch.zeros(128, 8, dtype=torch.bfloat16)},
              str(bad / checkpoint.SINGLE_FILE))
    with pytest.raises(ValueError, match="dtype"):
        checkpoint.read_projection(checkpoint.CheckpointIndex.from_model_dir(str(bad)), 0,
                                   range(0, 1), "up_proj", 128, 256)
    # an index whose weight_map is missing or malformed
    with pytest.raises(ValueError, match="weight_map"):
        checkpoint.CheckpointIndex.from_index_json(str(tmp_path), {"metadata": {}})
    with pytest.raises(ValueError, match="shard string"):
        checkpoint.CheckpointIndex.from_index_json(str(tmp_path), {"weight_map": {"a": 1}})
    with pytest.raises(FileNotFoundError):
        checkpoint.CheckpointIndex.from_model_dir(str(tmp_path / "nowhere"))
    # the index names a shard that does not hold the tensor
    idx = json.load(open(tmp_path / checkpoint.INDEX_FILE))
    n0 = checkpoint.expert_tensor_name(3, 0, "gate_proj", "weight_packed")
    idx["weight_map"][n0] = "model-00002-of-00002.safetensors"
    moved = checkpoint.CheckpointIndex.from_index_json(str(tmp_path), idx)
    with pytest.raises(KeyError, match="not in"):
        checkpoint.read_projection(moved, 3, range(0, 1), "gate_proj", 128, 256)
