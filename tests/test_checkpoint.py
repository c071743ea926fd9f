"""The checkpoint reader and upload plan on the CPU: the reference's own tests of
src/checkpoint/file.rs:138-205 and src/checkpoint/plan.rs:266-359, on synthetic
checkpoints written by tests/ckpt_fixture.py (the reference's need a local Krea 2 model)."""

import numpy as np
import pytest

import krea2_w8a8 as k2
from ckpt_fixture import block_tensors, expected_layout, write_raw, write_safetensors
from krea2_w8a8.checkpoint import Checkpoint, Plan


def test_a_file_that_is_not_safetensors_is_refused_by_name():
    with pytest.raises(k2.InvalidArgument, match=r"not a ComfyUI checkpoint \(.safetensors\)"):
        Checkpoint("/models/krea2.bin")


def test_a_header_longer_than_the_file_is_refused(tmp_path):
    path = tmp_path / "long.safetensors"
    write_raw(path, "{}", b"", length=2**64 - 1)
    with pytest.raises(k2.InvalidArgument, match="^cannot read "):
        Checkpoint(path)


def test_a_tensor_reaching_past_the_data_is_refused(tmp_path):
    path = tmp_path / "span.safetensors"
    write_raw(path, '{"w":{"dtype":"I8","shape":[2,2],"data_offsets":[0,64]}}', bytes(4))
    with pytest.raises(k2.InvalidArgument, match="^cannot read "):
        Checkpoint(path)


def test_a_size_that_disagrees_with_dtype_and_shape_is_refused(tmp_path):
    path = tmp_path / "size.safetensors"
    write_raw(path, '{"w":{"dtype":"F32","shape":[2,2],"data_offsets":[0,4]}}', bytes(4))
    with pytest.raises(k2.InvalidArgument, match="^cannot read "):
        Checkpoint(path)


def test_tensors_read_back_with_their_dtype_shape_and_bytes(tmp_path):
    path = tmp_path / "read.safetensors"
    header = ('{"__metadata__":{"format":"pt"},'
              '"w":{"dtype":"I8","shape":[2,3],"data_offsets":[0,6]},'
              '"s":{"dtype":"F32","shape":[2],"data_offsets":[6,14]}}')
    write_raw(path, header, bytes([1, 2, 3, 4, 5, 6]) + bytes(8))
    with Checkpoint(path) as f:
        w = f.get("w")
        assert (w.dtype, w.shape) == ("I8", (2, 3))
        assert w.numpy().tolist() == [[1, 2, 3], [4, 5, 6]]
        assert f.get("s").dtype == "F32"
        with pytest.raises(k2.InvalidArgument, match="^missing tensor __metadata__ in "):
            f.get("__metadata__")
        with pytest.raises(k2.InvalidArgument, match="^missing tensor missing in "):
            f.get("missing")


def test_a_whole_model_save_reads_under_the_transformer_names(tmp_path):
    path = tmp_path / "wrapped.safetensors"
    header = ('{"__metadata__":{"workflow":"{}"},'
              '"model.diffusion_model.blocks.0.attn.wq.weight":{"dtype":"I8","shape":[1],"data_offsets":[0,1]},'
              '"model.diffusion_model.first.weight":{"dtype":"I8","shape":[1],"data_offsets":[1,2]}}')
    write_raw(path, header, bytes([7, 9]))
    with Checkpoint(path) as f:
        assert f.get("first.weight").numpy().tolist() == [9]
        assert f.block_count() == 1
        with pytest.raises(k2.InvalidArgument):
            f.get("model.diffusion_model.first.weight")


def test_block_count_takes_only_the_decimal_form_of_each_index(tmp_path):
    # src/checkpoint/file.rs:115-119 looks up exactly `blocks.{i}.attn.wq.weight` for
    # i = 0, 1, ...: `blocks.01` is not block 1, and `blocks.+1` / `blocks. 1` are no
    # blocks at all, so this file holds one block.
    path = tmp_path / "zeros.safetensors"
    names = ["blocks.0.attn.wq.weight", "blocks.01.attn.wq.weight", "blocks.+1.attn.wq.weight",
             "blocks.00.attn.wq.weight"]
    header = "{" + ",".join(
        f'"{n}":{{"dtype":"I8","shape":[1],"data_offsets":[{i},{i + 1}]}}' for i, n in enumerate(names)) + "}"
    write_raw(path, header, bytes(len(names)))
    with Checkpoint(path) as f:
        assert f.block_count() == 1


def test_names_without_a_shared_wrapper_are_kept(tmp_path):
    path = tmp_path / "mixed.safetensors"
    header = ('{"model.blocks.0.attn.wq.weight":{"dtype":"I8","shape":[1],"data_offsets":[0,1]},'
              '"first.weight":{"dtype":"I8","shape":[1],"data_offsets":[1,2]}}')
    write_raw(path, header, bytes([7, 9]))
    with Checkpoint(path) as f:
        f.get("model.blocks.0.attn.wq.weight")
        f.get("first.weight")


@pytest.fixture(scope="module")
def synthetic(tmp_path_factory):
    rng = np.random.default_rng(5)
    t = block_tensors(rng, layers=2)
    path = tmp_path_factory.mktemp("ckpt") / "krea2_synthetic.safetensors"
    write_safetensors(path, t, metadata={"format": "pt"})
    return path, t


def test_the_plan_lays_out_the_blocks(synthetic):
    path, t = synthetic
    with Checkpoint(path) as f:
        plan = Plan(f)
        assert plan.layers == 2 == f.block_count()
        qkvg = plan.span("blocks.0.qkvg.q")
        assert qkvg.rows == 256 + 64 + 64 + 256
        assert (qkvg.row_bytes, qkvg.device_row_bytes, qkvg.segments) == (256, 256, 4)
        # 8192-byte rows take one 64-byte step of pitch padding (src/kernels/shape.rs:105-107).
        down = plan.span("blocks.0.down.q")
        assert (down.rows, down.row_bytes, down.device_row_bytes) == (256, 8192, 8256)
        assert down.device_bytes == 256 * 8256 and down.file_bytes == 256 * 8192
        spans = sorted((plan.span(n) for n in plan.names()), key=lambda s: s.device_offset)
        end = 0
        for span in spans:
            assert span.device_offset % 256 == 0 and span.device_offset >= end
            end = span.device_offset + span.device_bytes
        assert plan.total_bytes >= end
        # offsets are assigned in name order
        offsets = [plan.span(n).device_offset for n in plan.names()]
        assert plan.names() == sorted(plan.names()) and offsets == sorted(offsets)
        assert set(plan.names()) == set(expected_layout(t, 2))


def test_the_gate_and_up_rows_interleave_in_sixteens(synthetic):
    path, _ = synthetic
    with Checkpoint(path) as f:
        plan = Plan(f)
        gu = plan.span("blocks.0.gu.q")
        assert gu.rows == 2 * 8192 and gu.segments == gu.rows // 16
        assert plan.span("blocks.0.gu.s").file_bytes == gu.rows * 4


def test_missing_or_malformed_block_tensors_are_refused(tmp_path):
    rng = np.random.default_rng(6)
    t = block_tensors(rng, layers=1, inter=256)
    broken = dict(t)
    del broken["blocks.0.mlp.up.weight_scale"]
    path = tmp_path / "broken.safetensors"
    write_safetensors(path, broken)
    with Checkpoint(path) as f, pytest.raises(k2.InvalidArgument, match="missing tensor blocks.0.mlp.up.weight_scale"):
        Plan(f)
    odd = dict(t)
    odd["blocks.0.mlp.up.weight"] = odd["blocks.0.mlp.up.weight"][:250]
    odd["blocks.0.mlp.up.weight_scale"] = odd["blocks.0.mlp.up.weight_scale"][:250]
    path = tmp_path / "odd.safetensors"
    write_safetensors(path, odd)
    with Checkpoint(path) as f, pytest.raises(k2.InvalidArgument, match="blocks.0.gu takes its parts 16 rows at a time in turn"):
        Plan(f)
    path = tmp_path / "empty.safetensors"
    write_safetensors(path, {"x": np.zeros(4, np.float32)})
    with Checkpoint(path) as f, pytest.raises(k2.InvalidArgument, match="no transformer blocks"):
        Plan(f)
