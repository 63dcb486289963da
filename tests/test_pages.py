"""PageArena (the native qx_pages_* accounting) and the oracle's restatement
against the reference's arena known answers, kept as data in
tests/golden/arena_known_answers.json (tests/engine/test_arena.py:10-138),
plus seeded property checks: no page is ever held by two keys and none
leaks, and the free stack hands pages out in order."""

import json
import random
from pathlib import Path

import pytest

from oracle import pages_ref
from quail_amd.pages import PageArena

GOLDEN = json.loads((Path(__file__).parent / "golden" / "arena_known_answers.json").read_text())
ARENAS = {"native": PageArena, "oracle": pages_ref.RefPageArena}

# reads of arena state by name: (arena, args) -> value
READS = {
    "free_pages": lambda a: a.free_pages,
    "resident_tokens": lambda a: a.resident_tokens,
    "retained_pages": lambda a: a.retained_pages,
    "retained_prefix_tokens": lambda a: a.retained_prefix_tokens,
    "owned": lambda a, key: a.owned[key],
    "tokens": lambda a, key: a.tokens[key],
    "retained": lambda a, key: a.retained[key],
    "borrowed": lambda a, key: a.borrowed[key],
    "pinned_contains": lambda a, key: key in a.pinned,
    "pinned_size": lambda a: len(a.pinned),
    "retained_size": lambda a: len(a.retained),
}
EXCEPTIONS = {"KeyError": KeyError, "ValueError": ValueError}


class Run:
    """Interpreter of one scenario's ops over one arena."""

    def __init__(self, arena):
        self.arena = arena
        self.bound = {}

    def value(self, spec):
        """Evaluate {op, args, kw, slice, index} (nested ops evaluated first)."""
        args = [self.value(x) if isinstance(x, dict) else x for x in spec.get("args", [])]
        kw = {k: self.value(v) if isinstance(v, dict) else v for k, v in spec.get("kw", {}).items()}
        op = spec["op"]
        if op in READS:
            out = READS[op](self.arena, *args)
        else:
            out = getattr(self.arena, op)(*args, **kw)
        if isinstance(out, tuple):
            out = list(out)
        if "slice" in spec:
            lo, hi = spec["slice"]
            out = list(out)[lo:hi]
        if "index" in spec:
            out = list(out)[spec["index"]]
        return out

    def step(self, spec):
        expect = spec.get("expect", {})
        if "raises" in expect:
            with pytest.raises(EXCEPTIONS[expect["raises"]]):
                self.value(spec)
            return
        out = self.value(spec)
        if "bind" in spec:
            self.bound[spec["bind"]] = list(out)
        where = f"{spec['op']}{tuple(spec.get('args', []))}"
        if "value" in expect:
            assert _plain(out) == expect["value"], where
        if "not" in expect:
            assert out is not expect["not"], where
        if "len" in expect:
            assert len(out) == expect["len"], where
        if "concat" in expect:
            want = []
            for name, lo, hi in expect["concat"]:
                want += self.bound[name][lo:hi]
            assert list(out) == want, where
        if "same_as" in expect:
            assert _plain(out) == _plain(self.value(expect["same_as"])), where


def _plain(x):
    if isinstance(x, (list, tuple)):
        return [_plain(v) for v in x]
    if hasattr(x, "tolist"):
        return x.tolist()
    return x


@pytest.mark.parametrize("impl", sorted(ARENAS))
@pytest.mark.parametrize("scenario", GOLDEN["scenarios"], ids=lambda s: s["name"])
def test_reference_arena_known_answers(scenario, impl):
    pages, page_tokens = scenario["arena"]
    run = Run(ARENAS[impl](num_pages=pages, page_tokens=page_tokens))
    for spec in scenario["ops"]:
        run.step(spec)


def test_known_answers_cover_the_reference_scenarios():
    """Every arena the reference test builds has its scenario (the random
    walk, an invariant rather than a known answer, is the property test
    below)."""
    sizes = [tuple(s["arena"]) for s in GOLDEN["scenarios"]]
    assert sizes == [(10, 16), (3, 4), (10, 4), (4, 16), (2, 16), (10, 16)]
    assert sum(len(s["ops"]) for s in GOLDEN["scenarios"]) >= 70


@pytest.mark.parametrize("impl", sorted(ARENAS))
def test_free_stack_hands_out_pages_in_order(impl):
    """Pages come off the free stack P-1 .. 0 from its top: a fresh arena
    gives 0, 1, 2, ..., and freed pages are the next ones handed out."""
    a = ARENAS[impl](num_pages=10, page_tokens=16)
    assert list(a.alloc("a", 40)) == [0, 1, 2]
    assert list(a.alloc("b", 20)) == [3, 4]
    a.free_key("a")
    assert sorted(a.alloc("c", 48)) == [0, 1, 2]


@pytest.mark.parametrize("seed", [5, 11, 23])
@pytest.mark.parametrize("impl", sorted(ARENAS))
def test_random_alloc_free_never_double_owns_or_leaks(impl, seed):
    rng = random.Random(seed)
    a = ARENAS[impl](num_pages=64, page_tokens=16)
    live = {}
    for step in range(400):
        if live and rng.random() < 0.45:
            key = rng.choice(sorted(live))
            a.free_key(key)
            del live[key]
        else:
            key = ("doc", step)
            got = a.alloc(key, rng.randrange(1, 200))
            if got is not None:
                live[key] = list(got)
        held = [p for pages in live.values() for p in pages]
        assert len(held) == len(set(held))
        assert len(held) + a.free_pages == 64
