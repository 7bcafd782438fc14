"""CPU: the pack reader (xl_pack_meta_get / xl_pack_types) on packs written in
the reference's layout, and its error paths. The device load is in
tests/test_gpu_pack.py."""
from __future__ import annotations

import os

import numpy as np
import pytest

import crosslane_amd as xl
from tests.packs import write_pack

SIGS = [(16, 16, 17), (29, 29, 29), (17, 17, 29), (16, 16, 16)]


def test_meta_and_types(orc, tmp_path):
    p = write_pack(str(tmp_path / "pack"), orc, SIGS, 256, 512, 4, seed=3)
    assert xl.pack_meta(p) == {"dim": 256, "ff": 512, "n_layers": 4, "n_experts": 4, "top_k": 6, "swiglu_limit": 0.0}
    q = write_pack(str(tmp_path / "pack_lim"), orc, SIGS[:1], 256, 256, 1, seed=3, swiglu_limit=7)
    assert xl.pack_meta(q)["swiglu_limit"] == 7.0
    ds4 = open(os.path.join(q, "ds4.txt")).read()
    open(os.path.join(q, "ds4.txt"), "w").write(ds4.replace("swiglu_limit 7", "swiglu_limit seven"))
    with pytest.raises(xl.XLError, match="swiglu_limit"):
        xl.pack_meta(q)
    t = xl.pack_types(p, 1, 3, 4)
    for l in range(3):
        assert (t[l] == np.array(SIGS[l + 1], np.int32)).all()


def test_reader_errors(orc, tmp_path):
    p = write_pack(str(tmp_path / "pack"), orc, SIGS[:2], 256, 256, 2, seed=3)
    with pytest.raises(xl.XLError, match="missing"):
        xl.pack_types(p, 0, 2, 3)                         # expert 2 is not in the pack
    with pytest.raises(xl.XLError, match="cannot read"):
        xl.pack_meta(str(tmp_path / "nowhere"))
    txt = open(os.path.join(p, "tensors.txt")).read()
    open(os.path.join(p, "tensors.txt"), "w").write(txt.replace(" IQ1_M ", " Q4_K ", 1))
    with pytest.raises(xl.XLError, match="not IQ2_XXS"):
        xl.pack_types(p, 0, 2, 2)
    open(os.path.join(p, "tensors.txt"), "w").write(txt + txt.splitlines()[-1] + "\n")
    with pytest.raises(xl.XLError, match="duplicate"):
        xl.pack_meta(p)
    open(os.path.join(p, "tensors.txt"), "w").write(txt)
    ds4 = open(os.path.join(p, "ds4.txt")).read()
    open(os.path.join(p, "ds4.txt"), "w").write(ds4.replace("format gguf", "format safetensors"))
    with pytest.raises(xl.XLError, match="gguf"):
        xl.pack_meta(p)
