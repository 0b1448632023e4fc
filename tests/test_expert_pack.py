"""Expert packs in the reference's format (include/vastloom/inference/deepseek_v4_expert_pack.hpp:
17-77; tools/pack_deepseek_experts.py:211-260): a written pack reads back byte for byte, records are
4 KiB aligned and in catalog-bundle tensor order (down, gate, up), and the structural checks the
reference's verifier makes on records refuse corrupt packs (tests/test_deepseek_expert_pack.cpp)."""

from __future__ import annotations

import json

import numpy as np
import pytest

from vastloom_amd import expert_pack as xp
from vastloom_amd.workloads import IQ2_XXS, Q8_0, random_matrix


def _experts(rng, ids, H=512, F=256):
    out = {}
    for e in ids:
        out[e] = {"gate": (IQ2_XXS, F, H, random_matrix(rng, IQ2_XXS, F, H, 0.01)),
                  "up": (IQ2_XXS, F, H, random_matrix(rng, IQ2_XXS, F, H, 0.01)),
                  "down": (Q8_0, H, F, random_matrix(rng, Q8_0, H, F, 0.01))}
    return out


def test_round_trip(tmp_path):
    experts = _experts(np.random.default_rng(0), [3, 0, 17])
    m = xp.write_pack(tmp_path, 5, experts)
    assert m["format"] == xp.FORMAT and m["layer"] == 5 and m["alignment"] == 4096
    assert [r["expert"] for r in m["experts"]] == [0, 3, 17]
    for r in m["experts"]:
        assert r["offset"] % 4096 == 0
        assert [t["name"].split(".")[2] for t in r["tensors"]] == ["ffn_down_exps", "ffn_gate_exps", "ffn_up_exps"]
        assert r["tensors"][0]["name"] == f"blk.5.ffn_down_exps.weight.expert.{r['expert']}"
    pack = xp.ExpertPack(tmp_path)
    assert pack.layer == 5 and sorted(pack.experts) == [0, 3, 17]
    for e, mats in experts.items():
        for p, (qtype, rows, cols, data) in mats.items():
            got = pack.experts[e].matrix(p)
            assert got[:3] == (qtype, rows, cols)
            assert np.array_equal(got[3], data)


def _corrupt(tmp_path, edit):
    xp.write_pack(tmp_path, 0, _experts(np.random.default_rng(1), [0, 1]))
    path = tmp_path / xp.MANIFEST_NAME
    m = json.loads(path.read_text())
    edit(m, tmp_path)
    path.write_text(json.dumps(m))


@pytest.mark.parametrize("case", ["format", "alignment", "misaligned", "overlap", "hash", "tensor_order",
                                  "missing_projection", "payload_size"])
def test_structural_refusals(tmp_path, case):
    def edit(m, root):
        r0, r1 = m["experts"]
        if case == "format":
            m["format"] = "vastloom.deepseek-v4-expert-pack.v0"
        elif case == "alignment":
            m["alignment"] = 512
        elif case == "misaligned":
            r1["offset"] += 64
        elif case == "overlap":
            r1["offset"] = r0["offset"]
        elif case == "hash":
            r0["sha256"] = "0" * 64
        elif case == "tensor_order":
            r0["tensors"][1]["packed_offset"] += 1
        elif case == "missing_projection":
            r0["tensors"][2]["name"] = r0["tensors"][2]["name"].replace("ffn_up_exps", "ffn_gate_exps")
        elif case == "payload_size":
            m["payload"]["bytes"] += 1
    _corrupt(tmp_path, edit)
    with pytest.raises(xp.PackError):
        xp.ExpertPack(tmp_path)
