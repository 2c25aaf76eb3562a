"""FP8 checkpoint format (inference/fp8_checkpoint.py:26-85, export_fp8.py:15-44)
on the host: the writer keeps every non-linear tensor, replaces each quantized
linear's weight by e4m3 codes plus a float32 `<name>.weight_scale`, and the
loader puts codes and scales back into FP8Linear buffers bit for bit. Most
tests pass the oracle's restatement as the quantizer; the export test runs the
product's own path on this GPU-less host (the library's host quantizer), as the
reference's exporter runs on the CPU (the GPU round trip is
tests/test_gpu_checkpoint.py)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
import torch.nn as nn
from safetensors import safe_open
from safetensors.torch import save_file

import oracle
from jeeves_amd import export_fp8, fp8_checkpoint
from jeeves_amd.fp8 import FP8Linear
from jeeves_amd.fp8_weights import FP8, SCALE_SUFFIX, replace_linears


def oracle_quantize(weight: torch.Tensor):
    codes, scale = oracle.quantize_rows(weight.float().numpy())
    return torch.from_numpy(codes).view(FP8), torch.from_numpy(scale)


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.q = nn.Linear(256, 1024, bias=False)     # quantizable
        self.o = nn.Linear(512, 1040, bias=True)      # quantizable, with bias
        self.head = nn.Linear(256, 256, bias=False)   # out < 1024: stays bf16
        self.norm = nn.LayerNorm(256)


def make_checkpoint(path, seed=0):
    g = torch.Generator().manual_seed(seed)
    tensors = {
        "q.weight": (torch.randn(1024, 256, generator=g) * 0.02).to(torch.bfloat16),
        "o.weight": (torch.randn(1040, 512, generator=g) * 0.02).to(torch.bfloat16),
        "o.bias": torch.randn(1040, generator=g).to(torch.bfloat16),
        "head.weight": torch.randn(256, 256, generator=g).to(torch.bfloat16),
        "norm.weight": torch.randn(256, generator=g).to(torch.bfloat16),
        "norm.bias": torch.randn(256, generator=g).to(torch.bfloat16),
    }
    save_file(tensors, str(path), metadata={"format": "pt"})
    return tensors


def test_quantized_linears_follow_the_reference_rule():
    assert fp8_checkpoint.quantized_linears(Block()) == {"q", "o"}


def test_write_quantized_format(tmp_path):
    src, dst = tmp_path / "in.safetensors", tmp_path / "out.safetensors"
    tensors = make_checkpoint(src)
    sizes = fp8_checkpoint.write_quantized(src, dst, {"q", "o"}, quantize=oracle_quantize)
    with safe_open(str(dst), framework="pt", device="cpu") as fh:
        keys = set(fh.keys())
        assert keys == set(tensors) | {"q.weight" + SCALE_SUFFIX, "o.weight" + SCALE_SUFFIX}
        for name in ("q", "o"):
            codes, scale = fh.get_tensor(f"{name}.weight"), fh.get_tensor(f"{name}.weight{SCALE_SUFFIX}")
            assert codes.dtype == FP8 and scale.dtype == torch.float32 and scale.shape == (codes.shape[0],)
            want_codes, want_scale = oracle.quantize_rows(tensors[f"{name}.weight"].float().numpy())
            assert np.array_equal(codes.view(torch.uint8).numpy(), want_codes)
            assert np.array_equal(scale.numpy().view(np.uint32), want_scale.view(np.uint32))
        for key in ("o.bias", "head.weight", "norm.weight", "norm.bias"):
            assert torch.equal(fh.get_tensor(key), tensors[key])
    assert sizes["q.weight"] == 1024 * 256 and sizes["q.weight" + SCALE_SUFFIX] == 1024 * 4


def fp8_block():
    m = Block().to(torch.bfloat16)
    replace_linears(m, lambda lin: FP8Linear(lin.in_features, lin.out_features, bias=lin.bias is not None))
    return m


def test_load_tensors_round_trip(tmp_path):
    src, dst = tmp_path / "in.safetensors", tmp_path / "out.safetensors"
    tensors = make_checkpoint(src)
    fp8_checkpoint.write_quantized(src, dst, {"q", "o"}, quantize=oracle_quantize)
    m = fp8_block()
    assert isinstance(m.q, FP8Linear) and isinstance(m.o, FP8Linear) and isinstance(m.head, nn.Linear)
    loaded, unexpected = fp8_checkpoint.load_tensors(m, [dst], FP8Linear)
    assert unexpected == []
    # every buffer of a loaded FP8 linear counts as loaded, the kernels' tiled
    # copy included (inference/fp8_checkpoint.py:78 adds named_buffers())
    assert loaded == {"q.weight", "q.scale", "q.tiled_codes", "o.weight", "o.scale", "o.tiled_codes", "o.bias",
                      "head.weight", "norm.weight", "norm.bias"}
    want_codes, want_scale = oracle.quantize_rows(tensors["q.weight"].float().numpy())
    assert np.array_equal(m.q.codes().view(torch.uint8).numpy(), want_codes)
    assert np.array_equal(m.q.scale.numpy(), want_scale)
    assert torch.equal(m.o.bias, tensors["o.bias"]) and torch.equal(m.head.weight, tensors["head.weight"])


def test_load_tensors_reports_unused_keys_and_bad_shapes(tmp_path):
    src, dst = tmp_path / "in.safetensors", tmp_path / "out.safetensors"
    make_checkpoint(src)
    fp8_checkpoint.write_quantized(src, dst, {"q", "o"}, quantize=oracle_quantize)
    extra = tmp_path / "extra.safetensors"
    save_file({"stray.weight": torch.zeros(2), "lonely.weight" + SCALE_SUFFIX: torch.ones(3)}, str(extra))
    _, unexpected = fp8_checkpoint.load_tensors(fp8_block(), [dst, extra], FP8Linear)
    assert unexpected == ["stray.weight", "lonely.weight" + SCALE_SUFFIX]
    bad = tmp_path / "bad.safetensors"
    save_file({"q.weight": torch.zeros(1024, 128, dtype=FP8), "q.weight" + SCALE_SUFFIX: torch.ones(1024)}, str(bad))
    with pytest.raises(ValueError, match="checkpoint"):
        fp8_checkpoint.load_tensors(fp8_block(), [bad], FP8Linear)
    # map_key renames checkpoint keys onto the module tree and can drop keys
    _, unexpected = fp8_checkpoint.load_tensors(fp8_block(), [dst], FP8Linear,
                                                map_key=lambda k: None if k.startswith("norm") else k)
    assert unexpected == []


@pytest.mark.skipif(torch.cuda.is_available(), reason="exercises the exporter on a host without a GPU")
def test_export_layout(tmp_path):
    """export_fp8 end to end on a host without a GPU: the quantized tensors are
    the oracle's codes and scales bit for bit."""
    src, out = tmp_path / "export", tmp_path / "fp8"
    src.mkdir()
    make_checkpoint(src / "model-00001-of-00002.safetensors", 1)
    save_file({"lm_head.weight": torch.randn(1024, 256).to(torch.bfloat16)}, str(src / "model-00002-of-00002.safetensors"))
    (src / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {
        "q.weight": "model-00001-of-00002.safetensors", "lm_head.weight": "model-00002-of-00002.safetensors"}}))
    (src / "export.json").write_text(json.dumps({"step": 7}))
    (src / "config.json").write_text("{}")
    (src / "README.md").write_text("not copied")
    drafter = tmp_path / "drafter.safetensors"
    save_file({"delta_q.weight": torch.randn(1024, 256).to(torch.bfloat16)}, str(drafter))
    linears = tmp_path / "linears.json"
    linears.write_text(json.dumps(["base.q", "base.o", "base.lm_head", "delta_q"]))
    export_fp8.main([str(src), "--out", str(out), "--drafter", str(drafter), "--linears", str(linears)])
    assert json.loads((out / "export.json").read_text()) == {"step": 7, "precision": "fp8"}
    assert (out / "config.json").exists() and not (out / "README.md").exists()
    index = json.loads((out / "model.safetensors.index.json").read_text())
    assert index["weight_map"]["lm_head.weight" + SCALE_SUFFIX] == "model-00002-of-00002.safetensors"
    assert index["metadata"]["total_size"] > 0
    with safe_open(str(out / "drafter.safetensors"), framework="pt", device="cpu") as fh:
        assert fh.get_tensor("delta_q.weight").dtype == FP8
    source = make_checkpoint(tmp_path / "again.safetensors", 1)
    with safe_open(str(out / "model-00001-of-00002.safetensors"), framework="pt", device="cpu") as fh:
        for name in ("q", "o"):
            want_codes, want_scale = oracle_quantize(source[f"{name}.weight"])
            assert torch.equal(fh.get_tensor(f"{name}.weight").view(torch.uint8), want_codes.view(torch.uint8)), name
            assert torch.equal(fh.get_tensor(f"{name}.weight" + SCALE_SUFFIX), want_scale), name
    with pytest.raises(FileExistsError):
        export_fp8.main([str(src), "--out", str(out), "--linears", str(linears)])
