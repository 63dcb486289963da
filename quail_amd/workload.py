"""Seeded synthetic corpora of the benchmark configurations.

Each document is a row prompt: a shared instruction prefix followed by the
document's own tokens (ids uniform over the vocabulary). The AI function's
answer is read at the prompt's last row, packed as a one-token suffix after
the document prefix, so every document computes its own last token and may
borrow the shared prefix pages of its prefix-tree parent
(crates/quail-planner/src/inputs/prefix.rs:19-21, :33-44).

  tiny       16 docs, lengths U[16, 128], vocab 4096, 32-token prefix,
             one 2048-row pack; AI.IF on ids 10 (yes) / 11 (no)
  qwen3-4b   512 docs, lognormal(median 256, sigma 0.8) clipped [32, 2048],
             64-token prefix, 16384-row packs; AI.IF
  qwen3-8b   256 docs, lognormal(1500, 0.6) clipped [256, 8192], 96-token
             prefix, 32768-row packs; AI.CLASSIFY over 4 label ids
  qwen3-32b  2048 docs, lognormal(400, 0.8) clipped [32, 4096], 64-token
             prefix, 16384-row packs; AI.SCORE
"""

from dataclasses import dataclass

import numpy as np

from quail_amd.model import CONFIGS


@dataclass
class Workload:
    name: str
    model: str
    prompts: list          # per document: int64 token array, prefix included
    prefix_tokens: int
    chunk_budget: int
    function: str          # "if", "score" or "classify"
    label_ids: tuple       # (yes, no) or the classify label ids
    page_tokens: int = 16

    @property
    def documents(self) -> int:
        return len(self.prompts)

    def describe_lengths(self) -> str:
        """The document length distribution of the workload, in words."""
        kind = _SPECS[self.name]["lengths"]
        if kind[0] == "uniform":
            return f"lengths uniform {kind[1]}..{kind[2]} tokens"
        _, median, sigma, lo, hi = kind
        return f"lognormal({median}, {sigma}) clipped {lo}..{hi} tokens"

    def groups_input(self):
        """(prefixes, suffixes): the prompt less its last token, and that token."""
        prefixes = [p[:-1] for p in self.prompts]
        suffixes = [[p[-1:]] for p in self.prompts]
        return prefixes, suffixes


_SPECS = {
    "tiny": dict(model="tiny", docs=16, lengths=("uniform", 16, 128), prefix=32,
                 budget=2048, function="if", labels=(10, 11)),
    "qwen3-4b": dict(model="qwen3-4b", docs=512, lengths=("lognormal", 256, 0.8, 32, 2048),
                     prefix=64, budget=16384, function="if", labels=(10, 11)),
    "qwen3-8b": dict(model="qwen3-8b", docs=256, lengths=("lognormal", 1500, 0.6, 256, 8192),
                     prefix=96, budget=32768, function="classify", labels=(10, 11, 12, 13)),
    "qwen3-32b": dict(model="qwen3-32b", docs=2048, lengths=("lognormal", 400, 0.8, 32, 4096),
                      prefix=64, budget=16384, function="score", labels=(10, 11)),
}


def make_workload(name: str, seed: int = 0, documents: int | None = None) -> Workload:
    spec = _SPECS[name]
    cfg = CONFIGS[spec["model"]]
    rng = np.random.default_rng(seed)
    n = spec["docs"] if documents is None else documents
    prefix = rng.integers(0, cfg.vocab, spec["prefix"], dtype=np.int64)
    kind = spec["lengths"][0]
    if kind == "uniform":
        _, lo, hi = spec["lengths"]
        lengths = rng.integers(lo, hi + 1, n)
    else:
        _, median, sigma, lo, hi = spec["lengths"]
        lengths = np.clip(np.rint(rng.lognormal(np.log(median), sigma, n)), lo, hi)
    prompts = [np.concatenate([prefix, rng.integers(0, cfg.vocab, int(L), dtype=np.int64)])
               for L in lengths]
    return Workload(name=name, model=spec["model"], prompts=prompts,
                    prefix_tokens=spec["prefix"], chunk_budget=spec["budget"],
                    function=spec["function"], label_ids=spec["labels"])
