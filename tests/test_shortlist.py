"""The shortlist file format and the vocabulary guard (host logic, no GPU).

Mirrors the reference's own tests of ``cf/shortlist.py`` (tests/test_shortlist.py:28-87) on the
reference's packaged shortlist, which ships inside the package (chain_flow_amd/data/shortlist_qwen3_5.pt)
as the proposer's last-resort list.
"""
from __future__ import annotations

from pathlib import Path

import pytest
import torch

from chain_flow_amd import shortlist

FIXTURE = Path(__file__).resolve().parents[1] / "chain-flow_amd" / "chain_flow_amd" / "data" / "shortlist_qwen3_5.pt"
# content identity recorded for the reference's packaged list (sorted int32 ids)
PACKAGED_SHA = "42fb98262c247aaf79c860da979b048c96408c885416161c6e83c2a93cc6dbfb"


def test_packaged_shortlist_is_the_qwen35_vocab():
    ids, meta = shortlist.load(FIXTURE)
    assert meta["vocab_size"] == shortlist.PACKAGED_VOCAB
    assert meta["format"] == 1
    assert ids.numel() == shortlist.PACKAGED_ROWS
    assert int(ids.max()) < shortlist.PACKAGED_VOCAB and int(ids.min()) >= 0
    assert torch.equal(ids, torch.unique(ids))               # sorted and unique


def test_packaged_shortlist_is_int32_and_small():
    raw = torch.load(FIXTURE, map_location="cpu", weights_only=True)
    assert raw["ids"].dtype == torch.int32
    assert FIXTURE.stat().st_size < 400_000


def test_content_identity():
    ids, _ = shortlist.load(FIXTURE)
    assert shortlist.ids_content_sha(ids) == PACKAGED_SHA
    # the identity is of the content: order and dtype do not change it
    assert shortlist.ids_content_sha(ids.flip(0).long()) == PACKAGED_SHA


def test_guard_accepts_the_vocabulary_it_was_built_for():
    ids, meta = shortlist.load(FIXTURE)
    assert shortlist.check(ids, meta, shortlist.PACKAGED_VOCAB) is None


@pytest.mark.parametrize("v", [151936, 248319, 248321, 32000])
def test_guard_refuses_a_different_vocabulary(v):
    ids, meta = shortlist.load(FIXTURE)
    why = shortlist.check(ids, meta, v)
    assert why and str(v) in why and "248320" in why


def test_guard_falls_back_to_a_max_id_check_for_a_legacy_bare_tensor(tmp_path):
    p = tmp_path / "legacy.pt"
    torch.save(torch.tensor([0, 5, 999], dtype=torch.int64), p)
    ids, meta = shortlist.load(p)
    assert meta == {}
    assert shortlist.check(ids, meta, 1000) is None
    why = shortlist.check(ids, meta, 500)
    assert why and "999" in why and "no vocab_size metadata" in why


def test_save_load_roundtrip_and_resolve(tmp_path):
    ids = torch.tensor([7, 3, 3, 11, 0], dtype=torch.int64)
    p = shortlist.save(tmp_path / "s.pt", ids, vocab_size=16, tokenizer="t", note="n")
    got, meta = shortlist.load(p)
    assert got.tolist() == [0, 3, 7, 11]
    assert meta == {"format": 1, "vocab_size": 16, "tokenizer": "t", "note": "n"}
    assert shortlist.resolve(torch.tensor([5, -1, 20, 5, 2]), 16).tolist() == [2, 5]
    with pytest.raises(ValueError):
        shortlist.save(tmp_path / "bad.pt", [1, 16], vocab_size=16)


def test_synthetic_shortlist_shape():
    s = shortlist.synthetic(1000, 100, seed=2)
    assert s.dtype == torch.int32 and s.numel() == 100
    assert torch.equal(s, s.unique()) and int(s.max()) < 1000
    assert torch.equal(s, shortlist.synthetic(1000, 100, seed=2))
