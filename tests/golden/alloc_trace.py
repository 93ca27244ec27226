"""Seeded allocator traces shared by make_alloc_golden.py (which runs them on the reference's
allocator in the build container) and tests/test_host.py (which runs them on mini-inference_amd's).

Test infrastructure. A trace only calls the allocator's public API, the way the reference
scheduler drives it (engine/scheduler.py:89-125, engine/engine.py:289-298): admission with
``allocate(len(prompt), token_ids=prompt)``, ``lengths[slot] = len(prompt)`` and
``register_prefix`` after the prefill, ``ensure_capacity`` as a request grows, ``free`` when it
finishes or is preempted. Each event leaves an observation of what the allocator handed back;
a digest of it is what the fixture stores.
"""

from __future__ import annotations

import hashlib
import random

# Prefix-caching trace: pool and request shapes.
PREFIX_POOL = dict(num_blocks=400, block_size=16, max_seqs=64, max_len=2048)
PREFIX_EVENTS = 3000
PREFIX_SEED = 11
VOCAB = 50


def digest(obs) -> str:
    return hashlib.sha256(repr(obs).encode()).hexdigest()[:16]


def prefix_churn(cache, events: int = PREFIX_EVENTS, seed: int = PREFIX_SEED) -> list[str]:
    """Admit / grow / finish requests on ``cache`` (prefix caching enabled); returns one digest
    per event of (event, slot, its block table, its length, prefix hit tokens, free blocks)."""
    rng = random.Random(seed)
    prefixes = [[rng.randrange(VOCAB) for _ in range(rng.randint(20, 200))] for _ in range(4)]
    live: dict[int, list[int]] = {}  # slot -> token ids
    out = []
    for e in range(events):
        r = rng.random()
        if live and r < 0.3:
            slot = rng.choice(sorted(live))
            del live[slot]
            cache.free(slot)
            obs = ("free", slot)
        elif live and r < 0.65:
            slot = rng.choice(sorted(live))
            toks = live[slot]
            grow = [rng.randrange(VOCAB) for _ in range(rng.randint(1, 32))]
            if cache.ensure_capacity(slot, len(toks) + len(grow)):
                toks.extend(grow)
                cache.lengths[slot] = len(toks)
                obs = ("grow", slot, tuple(cache.block_tables[slot]), cache.lengths[slot])
            else:  # preempted: the scheduler frees it and recomputes it later
                del live[slot]
                cache.free(slot)
                obs = ("preempt", slot)
        else:
            prompt = list(rng.choice(prefixes)) + [rng.randrange(VOCAB) for _ in range(rng.randint(1, 100))]
            if cache.can_allocate(len(prompt)):
                slot = cache.allocate(len(prompt), token_ids=prompt)
                hit = cache.lengths[slot]
                cache.lengths[slot] = len(prompt)
                cache.register_prefix(slot, prompt)
                live[slot] = prompt
                obs = ("admit", slot, tuple(cache.block_tables[slot]), hit)
            else:
                obs = ("full",)
        out.append(digest((e, obs, cache.prefix_hit_tokens, cache.num_free_blocks)))
    return out
