"""Speculative decoding host loop (flint_amd/spec.py) on the CPU.

The accept / mask / compaction helpers are checked against brute force (transitive closure of the
parent relation, enumeration of every agreeing root-to-node path, replay of the reference's
one-at-a-time slot copies, spec_tree.py:126-128). The whole chain and tree loops (reference
spec_mega.py:89-117, spec_tree.py:85-133) run against a stand-in target model whose next token is
a function of the token context it reads back from its own cache slots, and which checks that
every cache slot it reads holds a row RoPE'd at that slot's position. The loop must emit exactly
the stand-in's sequential greedy tokens (reference result.md:111-113). The stand-in lives here
only: the package's Transformer runs on the HIP library and nothing else.
"""
import itertools

import numpy as np
import pytest
import torch

from flint_amd import _lib
from flint_amd.spec import (LookupDraft, SpecDecoder, accept_chain, accept_tree, compaction_moves,
                            tree_depths, tree_mask)


# ----------------------------------------------------------------------------- helpers

def _random_tree(rng, m):
    return [-1] + [int(rng.integers(0, i)) for i in range(1, m)]


def test_tree_mask_is_transitive_closure():
    rng = np.random.default_rng(0)
    for m in list(range(1, 17)) * 4:
        parents = _random_tree(rng, m)
        a = np.zeros((m, m), dtype=np.int64)          # a[i][p] = 1: p is i's parent
        for i in range(1, m):
            a[i, parents[i]] = 1
        closure = np.eye(m, dtype=np.int64)
        step = np.eye(m, dtype=np.int64)
        for _ in range(m):
            step = np.minimum(step @ a, 1)
            closure = np.minimum(closure + step, 1)
        assert np.array_equal(tree_mask(parents), closure.astype(np.uint8))
        # depth = number of strict ancestors
        assert tree_depths(parents) == list(closure.sum(1) - 1)


def test_chain_mask_is_causal():
    for m in range(1, 17):
        parents = list(range(-1, m - 1))
        assert np.array_equal(tree_mask(parents), np.tril(np.ones((m, m), dtype=np.uint8)))
        assert tree_depths(parents) == list(range(m))


@pytest.mark.parametrize("parents", [[0], [-1, 1], [-1, -1], [-1, 0, 3, 1], [-1, 0, 2]])
def test_tree_rejects_bad_parents(parents):
    with pytest.raises(ValueError):
        tree_depths(parents)


def _brute_accept(cand, parents, targets):
    """Longest path from the root whose every step takes the target's token at its parent."""
    m = len(cand)
    best = [0]
    for i in range(m):
        path = [i]
        while parents[path[0]] != -1:
            path.insert(0, parents[path[0]])
        if all(cand[path[s]] == targets[path[s - 1]] for s in range(1, len(path))):
            if len(path) > len(best):
                best = path
    return best


def test_accept_tree_matches_brute_force():
    rng = np.random.default_rng(1)
    for trial in range(400):
        m = int(rng.integers(1, 17))
        parents = _random_tree(rng, m)
        # distinct sibling tokens, so at most one agreeing child per node
        cand = [0] * m
        used = {}
        for i in range(1, m):
            sib = used.setdefault(parents[i], set())
            t = int(rng.integers(0, 6))
            while t in sib:
                t = (t + 1) % 6 if len(sib) < 6 else int(rng.integers(100, 200))
            sib.add(t)
            cand[i] = t
        cand[0] = int(rng.integers(0, 6))
        targets = [int(rng.integers(0, 6)) for _ in range(m)]
        assert accept_tree(cand, parents, targets) == _brute_accept(cand, parents, targets), trial


def test_accept_tree_first_matching_child_wins():
    # two children carry the target's token: the walk takes the first in node order
    cand = [5, 7, 7, 9]
    parents = [-1, 0, 0, 2]
    targets = [7, 1, 9, 0]
    assert accept_tree(cand, parents, targets) == [0, 1]


def test_accept_chain_equals_tree_walk_on_a_chain():
    rng = np.random.default_rng(2)
    for _ in range(300):
        k = int(rng.integers(0, 16))
        draft = [int(rng.integers(0, 3)) for _ in range(k)]
        targets = [int(rng.integers(0, 3)) for _ in range(k + 1)]
        cand = [9] + draft
        parents = list(range(-1, k))
        acc = accept_chain(targets, draft)
        assert accept_tree(cand, parents, targets) == list(range(acc + 1))


def test_compaction_equals_in_order_copies():
    """fl_kv_move reads every source row before writing any; the reference copies one row at a
    time in path order (spec_tree.py:126-128). Both give the same cache for every increasing path,
    and the moved rows land in slots pos..pos+L in path order."""
    rng = np.random.default_rng(3)
    for _ in range(300):
        m = int(rng.integers(1, 17))
        pos = int(rng.integers(0, 40))
        L = int(rng.integers(0, m))
        path = [0] + sorted(int(x) for x in rng.choice(np.arange(1, m), size=L, replace=False)) if L else [0]
        src, dst = compaction_moves(path, pos)
        assert all(s > d for s, d in zip(src, dst))
        base = np.arange(pos + m) * 10
        seq = base.copy()
        for s, d in zip(src, dst):
            seq[d] = seq[s]
        par = base.copy()
        par[dst] = base[src]
        assert np.array_equal(seq, par)
        for s in range(len(path)):
            assert par[pos + s] == base[pos + path[s]]


# ----------------------------------------------------------------------------- LookupDraft

def test_lookup_draft_chain_takes_most_recent_longest_match():
    d = LookupDraft(max_ngram=3, min_ngram=1)
    ctx = [1, 2, 3, 4, 9, 1, 2, 3, 5, 6, 7, 2, 3]
    # "2 3" last occurred before 5 (most recent), earlier before 4
    assert d.chain(ctx, None, 3) == [5, 6, 7]
    assert d.chain([1, 2, 3], None, 4) == []                 # no earlier occurrence
    assert d.chain([4, 4], None, 4) == [4]                   # continuation cut at the context end


def test_lookup_draft_tree_merges_continuations():
    d = LookupDraft(max_ngram=2, min_ngram=1, width=3, depth=3)
    ctx = [7, 1, 2, 3, 7, 1, 2, 4, 7, 1, 5, 7, 1]
    toks, pars = d.tree(ctx, None)
    # "7 1" was followed by 5 7 1 / 2 4 7 / 2 3 7 (most recent first); the 2 branches share a node
    assert toks == [5, 7, 1, 2, 4, 7, 3, 7]
    assert pars == [-1, 0, 1, -1, 3, 4, 3, 6]
    tree_depths([-1] + [p + 1 for p in pars])


def test_lookup_draft_tree_respects_node_cap():
    d = LookupDraft(max_ngram=1, width=8, depth=8, max_nodes=6)
    ctx = list(itertools.chain.from_iterable([[0, i, i + 1, i + 2] for i in range(1, 9)])) + [0]
    toks, pars = d.tree(ctx, None)
    assert len(toks) == 5
    tree_depths([-1] + [p + 1 for p in pars])


# ----------------------------------------------------------------------------- stand-in model

V = 37


def target_next(ctx):
    """The stand-in's greedy next token: mostly a function of the last two tokens (so drafts can
    guess it), every few positions a hash of the whole context (so any corrupted slot shows)."""
    n = len(ctx)
    if n % 3 == 0:
        h = 0
        for i, t in enumerate(ctx):
            h = (h * 1000003 + (t + 1) * (i + 11)) % (1 << 61)
        return h % V
    a = ctx[-1]
    b = ctx[-2] if n > 1 else 0
    return (5 * a + 3 * b + 1) % V


class _Cfg:
    vocab_size = V
    dim = 4


class StandInModel:
    """Implements the Transformer calls the spec loop and generate.prefill make (setup_caches,
    verify, decode_step, kv_move) over a cache of (token, rope position) rows."""
    device = torch.device("cpu")
    config = _Cfg()

    def __init__(self):
        self.slots = []
        self.moves = 0
        self.decodes = 0

    def setup_caches(self, b, s):
        self.slots = [None] * s
        self._prefill_masks = {}

    def _prefix(self, pos):
        out = []
        for s in range(pos):
            row = self.slots[s]
            assert row is not None and row[1] == s, f"slot {s} holds {row}"
            out.append(row[0])
        return out

    def verify(self, tokens, pos, depth=None, amask=None, logits=None, feat=None, tokens_out=None):
        toks = [int(t) for t in tokens.reshape(-1).tolist()]
        m = len(toks)
        assert 1 <= m <= _lib.MAX_VERIFY and pos + m <= len(self.slots)
        depth = depth.tolist()
        amask = amask.reshape(m, m).tolist()
        prefix = self._prefix(pos)
        tout = []
        for i in range(m):
            anc = [j for j in range(m) if amask[i][j]]
            assert anc[-1] == i and depth[i] == len(anc) - 1
            tout.append(target_next(prefix + [toks[j] for j in anc]))
            self.slots[pos + i] = (toks[i], pos + depth[i])
            if feat is not None and feat is not False:
                feat[i] = toks[i]
        out = torch.tensor(tout, dtype=torch.int32)
        if tokens_out is not None:
            tokens_out[:m] = out
            out = tokens_out
        return out, logits, feat

    def decode_step(self, token, pos, token_out=None, logits=None, feat=None):
        self.decodes += 1
        tout, _, _ = self.verify(token.reshape(1), pos, depth=torch.zeros(1, dtype=torch.int32),
                                 amask=torch.ones(1, 1, dtype=torch.uint8), feat=None if feat is None else feat.view(1, -1),
                                 tokens_out=token_out)
        return tout

    def kv_move(self, src, dst):
        assert len(src) == len(dst) <= _lib.MAX_VERIFY
        rows = [self.slots[s] for s in src]
        for d, r in zip(dst, rows):
            self.slots[d] = r
        self.moves += len(src)


def greedy(prompt, n):
    seq = list(prompt)
    for _ in range(n):
        seq.append(target_next(seq))
    return seq


class OracleDraft:
    """Knows the stand-in's rule: proposes the true continuation with planted mistakes (chain), or
    a tree whose true branch sits behind decoy siblings at a random position (tree). Also checks
    that the features handed to it are those of the verified tokens, in order."""

    def __init__(self, prompt, seed, err=0.2, width=3, depth=5, max_nodes=16):
        self.rng = np.random.default_rng(seed)
        self.err, self.width, self.depth, self.max_nodes = err, width, depth, max_nodes
        self.t0 = len(prompt) - 1

    def _check_feats(self, context, feats):
        assert feats[:, 0].tolist() == [float(t) for t in context[self.t0:-1]]

    def chain(self, context, feats, k):
        self._check_feats(context, feats)
        ctx = list(context)
        out = []
        for _ in range(k):
            t = target_next(ctx)
            if self.rng.random() < self.err:
                t = (t + 1 + int(self.rng.integers(0, V - 1))) % V
            out.append(t)
            ctx.append(t)
        return out

    def tree(self, context, feats):
        self._check_feats(context, feats)
        toks, pars = [], []
        frontier = [(-1, list(context))]
        for _ in range(self.depth):
            nxt = []
            for par, ctx in frontier:
                true = target_next(ctx)
                kids = [int(x) for x in self.rng.choice(V, size=self.width, replace=False)]
                if true not in kids and self.rng.random() > self.err:
                    kids[int(self.rng.integers(0, self.width))] = true
                for t in kids:
                    if len(toks) >= self.max_nodes - 1:
                        return toks, pars
                    toks.append(t)
                    pars.append(par)
                    if t == true:
                        nxt.append((len(toks) - 1, ctx + [t]))
            frontier = nxt
            if not frontier:
                break
        return toks, pars


@pytest.mark.parametrize("mode", ["chain", "tree"])
@pytest.mark.parametrize("seed", range(6))
def test_spec_loop_equals_sequential_greedy(mode, seed):
    rng = np.random.default_rng(100 + seed)
    prompt = [int(x) for x in rng.integers(0, V, size=int(rng.integers(1, 30)))]
    n = 80
    model = StandInModel()
    draft = OracleDraft(prompt, seed)
    out, st = SpecDecoder(model, draft, k=int(rng.integers(1, 9))).generate(prompt, n, mode=mode)
    assert out == greedy(prompt, n)
    assert st.tokens == n and st.passes < n
    if mode == "tree":
        assert model.moves > 0           # some accepted nodes sat behind decoys


@pytest.mark.parametrize("mode", ["chain", "tree"])
def test_spec_loop_with_lookup_and_useless_drafts(mode):
    prompt = [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5]
    for draft in (LookupDraft(width=3, depth=5), OracleDraft(prompt, 9, err=1.0)):
        model = StandInModel()
        out, st = SpecDecoder(model, draft, k=6).generate(prompt, 64, mode=mode)
        assert out == greedy(prompt, 64)


def test_spec_loop_k0_eos_and_lengths():
    prompt = [1, 2, 3]
    ref = greedy(prompt, 50)
    model = StandInModel()
    out, st = SpecDecoder(model, OracleDraft(prompt, 0), k=0).generate(prompt, 50)
    assert out == ref and st.passes == 49          # one pass per token after the first
    assert model.decodes == 50                     # a lone root goes through the decode step
    eos = ref[len(prompt) + 20]
    stop = ref.index(eos, len(prompt))
    for mode in ("chain", "tree"):
        out, _ = SpecDecoder(StandInModel(), OracleDraft(prompt, 1, err=0.0), k=7).generate(
            prompt, 50, mode=mode, eos=eos)
        assert out == ref[:stop + 1]
    out, st = SpecDecoder(StandInModel(), OracleDraft(prompt, 0)).generate(prompt, 0)
    assert out == prompt and st.passes == 0
    out, _ = SpecDecoder(StandInModel(), OracleDraft([7], 0)).generate([7], 5, mode="tree")
    assert out == greedy([7], 5)


def test_spec_loop_rejects_bad_drafts():
    class Bad:
        def __init__(self, toks, pars):
            self.r = (toks, pars)

        def chain(self, context, feats, k):
            return self.r[0]

        def tree(self, context, feats):
            return self.r

    with pytest.raises(ValueError):
        SpecDecoder(StandInModel(), Bad([V + 1], [-1])).generate([1, 2], 4)
    with pytest.raises(ValueError):
        SpecDecoder(StandInModel(), Bad([1, 2], [-1, 5])).generate([1, 2], 4, mode="tree")
    with pytest.raises(ValueError):
        SpecDecoder(StandInModel(), k=_lib.MAX_VERIFY)
    with pytest.raises(ValueError):
        SpecDecoder(StandInModel()).generate([], 4)


def test_lookup_draft_incremental_index_equals_fresh():
    """The n-gram index grows with the context the loop passes back (the same list, longer each
    pass) and is rebuilt for an unrelated context; proposals equal a fresh draft's every time."""
    rng = np.random.default_rng(7)
    ctx = [int(x) for x in rng.integers(0, 12, size=40)]
    d = LookupDraft(width=3, depth=4)
    for step in range(120):
        ctx.append(int(rng.integers(0, 12)))
        if step == 60:                                  # an unrelated context of another length
            other = [int(x) for x in rng.integers(0, 12, size=70)]
            assert d.tree(other, None) == LookupDraft(width=3, depth=4).tree(list(other), None)
        fresh = LookupDraft(width=3, depth=4)
        assert d.tree(ctx, None) == fresh.tree(list(ctx), None)
        assert d.chain(ctx, None, 5) == fresh.chain(list(ctx), None, 5)


def test_lookup_draft_reused_on_a_different_context():
    """A reused LookupDraft given a context that shares the previous one's length, first and last
    tokens but differs inside must propose what a fresh draft proposes (no stale n-gram
    positions), and SpecDecoder-style reset() returns it to a fresh state."""
    from flint_amd.spec import LookupDraft
    a = [1, 2, 3, 4, 5, 6, 7, 8, 9, 1, 2, 3, 4, 5, 6, 7, 8, 40, 41, 42, 1, 2, 3, 4, 5, 6, 7, 8]
    b = list(a)
    b[9:17] = [50, 51, 52, 53, 54, 55, 56, 57]         # same length, head and tail
    reused = LookupDraft(max_ngram=3, width=3, depth=4)
    reused.chain(a, None, 4)
    reused.tree(a, None)
    fresh = LookupDraft(max_ngram=3, width=3, depth=4)
    assert reused.chain(b, None, 4) == fresh.chain(b, None, 4)
    assert reused.tree(b, None) == LookupDraft(max_ngram=3, width=3, depth=4).tree(b, None)
    # extension of the indexed context keeps using (and extending) the index
    ext = b + [9, 1, 2]
    assert reused.chain(ext, None, 4) == LookupDraft(max_ngram=3, width=3, depth=4).chain(ext, None, 4)
    reused.reset()
    assert reused.tree(a, None) == LookupDraft(max_ngram=3, width=3, depth=4).tree(a, None)
