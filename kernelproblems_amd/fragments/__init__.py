"""Per-fragment drop-ins for the reference's hot-path fragments.

Each module ``<round>_<id>`` mirrors ``<round>/<id>/problem.py``: it exports
``kernel_function(*inputs)`` with the inputs of that fragment's
``Model.forward`` in the same order, returning the same outputs (dtype, shape,
aliasing between views), and ``get_inputs()`` drawing inputs of the same
shapes and strides.  ``load("v8/d8f596b3df34")`` returns the module.
"""
from __future__ import annotations

import importlib

_CANONICAL = (
    # RMSNorm forward
    "v7/59f786beb25f", "v8/4b90e2d83144", "v8/f4e9e58fef73", "v7/215dd2e6a519", "v6/ac3fb0b7281f",
    "v1/84496d824942", "v1/2a844503364a",
    # residual add + RMSNorm forward (+ FSDP parameter unshard)
    "v8/7884328a5557", "v8/8e33a91b7364", "v8/94985bdb7630", "v8/7815074de963", "v1/18b859c50de2",
    "v5/013a3088b488",
    # RMSNorm backward (+ gradient adds, + residual add recompute)
    "v7/45990c83cfd6", "v8/d8f596b3df34", "v7/7f544ceb2120", "v7/ed20955ec34b", "v8/3c6c589cdf81",
    "v8/43f0c930291e",
    # embedding forward / backward
    "v7/1e49beb8a123", "v8/12545c1e9b06", "v7/a12a160cb11b",
    # RoPE (interleaved complex, table) forward / backward
    "v7/e29b92927600", "v8/493cad38cac9", "v8/c8c60d8f7015", "v8/97032595d968", "v7/0f38bc55457c",
    "v7/5c65f62b0422", "v7/bfe872e373e4", "v5/ca76bd89ec38", "v4/6b92d6e665ab", "v6/03d64c25b654",
    "v6/dc55b25cdcb2", "v5/a1bb72d946b0", "v4/a1318bc813d2", "v6/c8c60d8f7015", "v8/7e38211c7f1c",
    # RoPE on complex64 q / k (the v1 captures)
    "v1/075cb40f3d5d", "v1/9cd8f72e74ce", "v1/f23f9bb4567a", "v1/d7efc428b2f5",
    # SwiGLU gate forward / backward (+ silu alone, forward recomputed with the backward)
    "v8/c68dae22972b", "v8/385e1beb9bb9", "v7/58e7a4d6cde3", "v4/65b4b565ed67", "v6/182d2dcd0652",
    "v5/441b7bf23822", "v4/c72358b8111e", "v5/c68dae22972b",
    # token cross-entropy forward / backward
    "v8/71f1d2c9f38b", "v8/622c35f5d1c6", "v7/e59c6b1b5156", "v5/fb5b36393cbd", "v4/80ad8e737b06",
    # chain: RMSNorm forward -> backward (+ gradient adds, residual) -> embedding backward
    "v6/0b493aad68f0", "v5/118d525f44e0", "v8/f6251e84e3fa",
    # chain: (residual add +) RMSNorm forward -> backward (+ gradient adds, residual epilogue)
    "v6/822931829090", "v6/e9198b707240", "v5/92ce4a0c7b2c", "v5/401b52261ef5", "v4/363b7b58c971",
    "v6/408ac0979ac5", "v4/9c745ea697a7", "v6/28b45679fca1", "v1/f7ad66842c19", "v5/ac7d64b3c769",
    "v5/cbfdd7549926", "v1/84c0a03c4374", "v1/680e4c57cdc8",
)

# Drop-ins that re-export another one: the fragment's problem.py computes the
# same outputs from the same inputs with only view / reshape / no-op
# view.dtype differences in its op sequence.
EQUIVALENT = {
    "v1/84496d824942": "v7/215dd2e6a519", "v1/18b859c50de2": "v8/8e33a91b7364",
    "v1/680e4c57cdc8": "v5/118d525f44e0", "v5/cbfdd7549926": "v4/9c745ea697a7",
    "v1/84c0a03c4374": "v5/401b52261ef5", "v5/ac7d64b3c769": "v1/f7ad66842c19",
    "v5/c68dae22972b": "v4/65b4b565ed67",
}


# Fragments whose problem.py is the op sequence of a canonical one above (same
# signature, outputs and input shapes; the rounds re-list a region under its
# id, some with view in place of reshape imports only): their modules
# re-export the canonical drop-in.
SAME_AS = {
    "v1/1e49beb8a123": "v7/1e49beb8a123", "v1/363b7b58c971": "v4/363b7b58c971", "v1/65b4b565ed67": "v4/65b4b565ed67",
    "v1/80ad8e737b06": "v4/80ad8e737b06", "v1/9c745ea697a7": "v4/9c745ea697a7", "v1/c72358b8111e": "v4/c72358b8111e",
    "v2/075cb40f3d5d": "v1/075cb40f3d5d", "v2/18b859c50de2": "v1/18b859c50de2", "v2/1e49beb8a123": "v7/1e49beb8a123",
    "v2/2a844503364a": "v1/2a844503364a", "v2/363b7b58c971": "v4/363b7b58c971", "v2/65b4b565ed67": "v4/65b4b565ed67",
    "v2/680e4c57cdc8": "v1/680e4c57cdc8", "v2/80ad8e737b06": "v4/80ad8e737b06", "v2/84496d824942": "v1/84496d824942",
    "v2/84c0a03c4374": "v1/84c0a03c4374", "v2/9c745ea697a7": "v4/9c745ea697a7", "v2/9cd8f72e74ce": "v1/9cd8f72e74ce",
    "v2/c72358b8111e": "v4/c72358b8111e", "v2/d7efc428b2f5": "v1/d7efc428b2f5", "v2/f23f9bb4567a": "v1/f23f9bb4567a",
    "v2/f7ad66842c19": "v1/f7ad66842c19", "v3/18b859c50de2": "v1/18b859c50de2", "v3/1e49beb8a123": "v7/1e49beb8a123",
    "v3/2a844503364a": "v1/2a844503364a", "v3/363b7b58c971": "v4/363b7b58c971", "v3/65b4b565ed67": "v4/65b4b565ed67",
    "v3/680e4c57cdc8": "v1/680e4c57cdc8", "v3/80ad8e737b06": "v4/80ad8e737b06", "v3/84496d824942": "v1/84496d824942",
    "v3/84c0a03c4374": "v1/84c0a03c4374", "v3/9c745ea697a7": "v4/9c745ea697a7", "v3/c72358b8111e": "v4/c72358b8111e",
    "v3/f7ad66842c19": "v1/f7ad66842c19", "v4/18b859c50de2": "v1/18b859c50de2", "v4/1e49beb8a123": "v7/1e49beb8a123",
    "v4/2a844503364a": "v1/2a844503364a", "v4/680e4c57cdc8": "v1/680e4c57cdc8", "v4/84496d824942": "v1/84496d824942",
    "v4/84c0a03c4374": "v1/84c0a03c4374", "v4/f7ad66842c19": "v1/f7ad66842c19", "v5/1e49beb8a123": "v7/1e49beb8a123",
    "v6/1e49beb8a123": "v7/1e49beb8a123", "v6/215dd2e6a519": "v7/215dd2e6a519", "v6/622c35f5d1c6": "v8/622c35f5d1c6",
    "v6/71f1d2c9f38b": "v8/71f1d2c9f38b", "v6/8e33a91b7364": "v8/8e33a91b7364", "v6/97032595d968": "v8/97032595d968",
    "v6/c68dae22972b": "v5/c68dae22972b", "v7/385e1beb9bb9": "v8/385e1beb9bb9", "v7/493cad38cac9": "v8/493cad38cac9",
    "v7/622c35f5d1c6": "v8/622c35f5d1c6", "v7/8e33a91b7364": "v8/8e33a91b7364", "v7/ac3fb0b7281f": "v6/ac3fb0b7281f",
    "v7/f4e9e58fef73": "v8/f4e9e58fef73", "v8/e29b92927600": "v7/e29b92927600",
}

FRAGMENTS = _CANONICAL + tuple(SAME_AS)


def module_name(fragment_id: str) -> str:
    return fragment_id.replace("/", "_")


def load(fragment_id: str):
    if fragment_id not in FRAGMENTS:
        raise KeyError(f"unknown fragment {fragment_id!r}")
    return importlib.import_module(f"{__name__}.{module_name(fragment_id)}")
