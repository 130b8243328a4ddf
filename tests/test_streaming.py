"""Streaming safetensors reader / writer (host side, no GPU)."""

from __future__ import annotations

import os

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file, save_file

from int_crush_converter_amd.streaming import SafetensorsIndex, StreamWriter


def _state():
    g = torch.Generator().manual_seed(0)
    return {"b.weight": torch.randn(5, 7, generator=g).to(torch.bfloat16),
            "a.bias": torch.randn(7, generator=g),
            "c.idx": torch.arange(9, dtype=torch.int64),
            "d.flag": torch.tensor([True, False]),
            "e.empty": torch.zeros(0, 3)}


def test_index_order_matches_load_file(tmp_path):
    p = str(tmp_path / "in.safetensors")
    st = _state()
    save_file(st, p, metadata={"x": "1"})
    idx = SafetensorsIndex(p)
    assert idx.names() == list(load_file(p).keys())
    assert idx.metadata == {"x": "1"}
    for n, t in st.items():
        assert torch.equal(idx.read(n), t), n


@pytest.mark.parametrize("reserve", [4096, 10])
def test_writer_roundtrip_and_header_overflow(tmp_path, reserve):
    # reserve 10: the header does not fit and the file is rewritten with it
    src = str(tmp_path / "in.safetensors")
    st = _state()
    save_file(st, src)
    idx = SafetensorsIndex(src)
    out = str(tmp_path / "out.safetensors")
    w = StreamWriter(out, reserve)
    w.add_file_copy("b.weight", idx)
    w.add_host("q", torch.arange(12, dtype=torch.uint8).reshape(3, 4))
    w.add_file_copy("a.bias", idx)
    w.add_host("s", torch.tensor([[1.5], [2.0]], dtype=torch.float16))
    w.add_file_copy("e.empty", idx)
    with pytest.raises(ValueError):
        w.add_host("q", torch.zeros(1))
    w.close({"int_crush.method": "int_crush"})
    assert not os.path.exists(out + ".partial")
    got = load_file(out)
    assert set(got) == {"b.weight", "q", "a.bias", "s", "e.empty"}
    assert torch.equal(got["b.weight"], st["b.weight"]) and torch.equal(got["a.bias"], st["a.bias"])
    assert torch.equal(got["q"], torch.arange(12, dtype=torch.uint8).reshape(3, 4))
    assert got["s"].dtype == torch.float16 and got["e.empty"].shape == (0, 3)
    with safe_open(out, framework="pt") as f:
        assert f.metadata() == {"int_crush.method": "int_crush"}


def test_writer_abort_leaves_nothing(tmp_path):
    out = str(tmp_path / "out.safetensors")
    w = StreamWriter(out, 1024)
    w.add_host("q", torch.zeros(4))
    w.abort()
    assert not os.path.exists(out) and not os.path.exists(out + ".partial")
