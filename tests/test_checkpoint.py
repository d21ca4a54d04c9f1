"""Checkpoints: safetensors files holding a tree of tensors (the reference's
python/rg/checkpoint.py format, pinned by its tests/test_framework.py:182-217)."""

import json
import os

import numpy as np
import pytest

import rustautograd_amd as rg


def test_round_trip_keeps_structure_dtypes_values_and_metadata(tmp_path):
    tree = {"w": rg.tensor([0.25, -1.5]), "stack": [rg.tensor([7, -8], "int32"), (rg.tensor(np.arange(6.0).reshape(2, 3)),)],
            "step": rg.tensor(12.0), "none": None}
    path = str(tmp_path / "ckpt.safetensors")
    rg.save(path, tree, metadata={"tokenizer": "byte", "note": "ünïcode ✓"})
    back, meta = rg.load(path, with_metadata=True)
    assert meta == {"tokenizer": "byte", "note": "ünïcode ✓"}
    assert rg.tree.structure(back) == rg.tree.structure(tree)
    for (n1, x), (n2, y) in zip(rg.tree.paths(tree), rg.tree.paths(back)):
        assert n1 == n2 and x.dtype == y.dtype and x.shape == y.shape and x.numpy().tobytes() == y.numpy().tobytes()
    assert not [f for f in os.listdir(tmp_path) if ".tmp." in f]
    assert rg.load(path)["stack"][1][0].tolist() == [[0.0, 1.0, 2.0], [3.0, 4.0, 5.0]]


def test_the_file_is_plain_safetensors_with_the_tree_in_its_metadata(tmp_path):
    path = str(tmp_path / "m.safetensors")
    rg.save(path, {"layer": {"w": rg.tensor([1.0, 2.0]), "b": rg.tensor([3], "int32")}, "n": [rg.tensor(4.0, "float64")]})
    raw = open(path, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + n])
    assert header["layer.b"] == {"dtype": "I32", "shape": [1], "data_offsets": [0, 4]}
    assert header["layer.w"] == {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}
    assert header["n.0"] == {"dtype": "F64", "shape": [], "data_offsets": [12, 20]}
    # The reference's encoding of the structure: null leaves, [kind, children], ["dict", keys, children].
    assert json.loads(header["__metadata__"]["rg_tree"]) == ["dict", ["layer", "n"], [["dict", ["b", "w"], [None, None]], ["list", [None]]]]
    body = raw[8 + n:]
    assert np.frombuffer(body[0:4], "<i4").tolist() == [3]
    assert np.frombuffer(body[4:12], "<f4").tolist() == [1.0, 2.0]
    assert np.frombuffer(body[12:20], "<f8").tolist() == [4.0]


def test_files_from_other_tools_load_as_flat_dicts_and_bare_leaves_as_value(tmp_path):
    foreign = str(tmp_path / "foreign.safetensors")
    h = json.dumps({"enc.w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}).encode()
    open(foreign, "wb").write(len(h).to_bytes(8, "little") + h + np.float32([7.0, -7.0]).tobytes())
    assert rg.load(foreign)["enc.w"].tolist() == [7.0, -7.0]
    single = str(tmp_path / "single.safetensors")
    rg.save(single, rg.tensor([1, 2, 3], "int32"))
    raw = open(single, "rb").read()
    assert "value" in json.loads(raw[8:8 + int.from_bytes(raw[:8], "little")])
    assert rg.load(single).tolist() == [1, 2, 3]


def test_corrupt_files_are_rejected(tmp_path):
    path = str(tmp_path / "m.safetensors")
    rg.save(path, {"a": rg.tensor(np.ones(16, np.float32))})
    raw = open(path, "rb").read()
    bad = str(tmp_path / "bad")
    for broken in (raw[:-4], raw[:5], (2 ** 60).to_bytes(8, "little") + raw[8:], raw[:8] + b"{not json" + raw[17:]):
        open(bad, "wb").write(broken)
        with pytest.raises(ValueError):
            rg.load(bad)
    header = json.loads(raw[8:8 + int.from_bytes(raw[:8], "little")])
    header["a"]["dtype"] = "BF16"
    h = json.dumps(header).encode()
    open(bad, "wb").write(len(h).to_bytes(8, "little") + h + raw[8 + int.from_bytes(raw[:8], "little"):])
    with pytest.raises(ValueError):
        rg.load(bad)
    with pytest.raises(TypeError):
        rg.save(path, {"a": rg.tensor([1.0])}, metadata={"n": 3})


def test_a_training_state_survives_a_checkpoint_and_resumes_identically(tmp_path):
    from rustautograd_amd import workloads
    step, state = workloads.gpt_train_step(workloads.GPT_CONFIGS["C3"]._replace(batch=2, block=16, layers=1))
    c = rg.compile(step, (state,), validate="none")
    first = rg.run(c, state, steps=3)
    path = str(tmp_path / "train.safetensors")
    rg.save(path, first.state, metadata={"steps": "3"})
    resumed = rg.run(c, rg.load(path), steps=2)
    straight = rg.run(c, state, steps=5)
    assert resumed.history["aux"] == straight.history["aux"][3:]
    for (n, x), (_, y) in zip(rg.tree.paths(resumed.state), rg.tree.paths(straight.state)):
        assert x.numpy().tobytes() == y.numpy().tobytes(), n
