"""The drafter's shortlist file: format, loading, the vocabulary guard and the content identity.

Same on-disk contract as the reference (``cf/shortlist.py:44-108, 220-223``): a torch-saved dict
``{"format": 1, "ids": int32[n] sorted unique, "vocab_size": V, "tokenizer": str, "note": str}``,
or a legacy bare tensor of ids.  ``check`` refuses a list built for another vocabulary instead of
clamping it; ``ids_content_sha`` names the list by its sorted int32 content.  Files are read with
``torch.load(weights_only=True)``, which executes nothing from the file.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import torch

PACKAGED_VOCAB = 248320
PACKAGED_ROWS = 62642
FORMAT = 1


def ids_content_sha(ids) -> str:
    """sha256 of the SORTED int32 ids: an identity for the list's content, not its file bytes."""
    t = ids if isinstance(ids, torch.Tensor) else torch.as_tensor(ids)
    return hashlib.sha256(t.to(torch.int32).flatten().sort().values.cpu().numpy().tobytes()).hexdigest()


def load(path):
    """``(ids int64 CPU tensor, meta dict)`` from a dict-format file or a legacy bare tensor."""
    obj = torch.load(str(path), map_location="cpu", weights_only=True)
    if isinstance(obj, dict):
        ids = obj["ids"]
        meta = {k: v for k, v in obj.items() if k != "ids"}
    else:
        ids, meta = obj, {}
    return ids.flatten().long(), meta


def check(ids, meta: dict, vocab_size: int):
    """``None`` if this list may be used against a ``vocab_size``-row head, else why not."""
    built = meta.get("vocab_size")
    if built is not None:
        if int(built) != int(vocab_size):
            return (f"built for vocab_size={int(built)} but this model's lm_head has "
                    f"{int(vocab_size)} rows -- the ids would name different tokens. If the list IS "
                    f"for this tokenizer, rebuild it with the model's head size "
                    f"(vocab_size={int(vocab_size)}), not the tokenizer's")
        return None
    mx = int(ids.max()) if ids.numel() else -1
    if mx >= int(vocab_size):
        return (f"contains token id {mx}, past this model's {int(vocab_size)}-row lm_head, and "
                f"carries no vocab_size metadata")
    return None


def resolve(ids: torch.Tensor, vocab_size: int) -> torch.Tensor:
    """The rows the head uses: in-range ids, deduplicated and sorted (the proposer's
    ``ids[(ids >= 0) & (ids < V)].unique()``), as int32."""
    ids = ids.flatten().long()
    return ids[(ids >= 0) & (ids < vocab_size)].unique().to(torch.int32)


def save(path, ids, vocab_size: int, tokenizer: str = "", note: str = ""):
    """Write a shortlist in the dict format (sorted unique int32 ids)."""
    ids = torch.as_tensor(ids).flatten().long().unique().to(torch.int32).contiguous()
    if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= vocab_size):
        raise ValueError(f"ids outside [0, {vocab_size})")
    torch.save({"format": FORMAT, "ids": ids, "vocab_size": int(vocab_size), "tokenizer": tokenizer,
                "note": note}, str(path))
    return Path(path)


def synthetic(vocab_size: int = PACKAGED_VOCAB, rows: int = PACKAGED_ROWS, seed: int = 2) -> torch.Tensor:
    """A seeded sorted shortlist of ``rows`` distinct ids (int32), the stand-in for a real one."""
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(vocab_size, generator=g)[:rows].sort().values.to(torch.int32)
