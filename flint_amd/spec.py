"""Speculative greedy decoding over fl_verify: the chain loop (reference spec_mega.py:89-117) and
the tree loop with KV compaction (reference spec_tree.py:85-133).

Each pass feeds the pending token (the root, not yet in the cache) plus a draft to one verify
launch at cache slots pos..pos+M-1, takes the target's greedy token per node (fl_verify's
on-device argmax), accepts the longest draft prefix (chain) or root-to-leaf path (tree) that the
target agrees with, and for a tree moves the accepted nodes' K/V rows into contiguous slots with
fl_kv_move. The emitted tokens equal sequential greedy decoding of the same model (reference
result.md:111-113), up to argmax ties that the verify and decode kernels break differently.

The draft is pluggable. The reference's EAGLE head (train/draft_model.py) is trained weights
and not part of this package; a draft here is any object with

    chain(context, feats, k) -> list[int]             up to k proposed tokens after context
    tree(context, feats)     -> (tokens, parents)      nodes below the root, parents[i] in
                                                        [-1, i) (-1 = the root), parents first

where context is every token so far (prompt, emitted tokens, and last the pending root) and feats
is a bf16 [n, dim] device view of the final-norm features of the verified tokens (the input an
EAGLE head consumes, reference spec_mega.py:112). LookupDraft (prompt-lookup n-gram matching)
needs no weights.
"""
import time

import numpy as np
import torch

from . import _lib
from .generate import prefill


def tree_depths(parents):
    """Depth of each node of a tree in verify order (node 0 = root, parents[0] = -1, every other
    parent an earlier node); raises ValueError on any other parent array. Reference
    spec_tree.py:98-100 builds the same depth list from the draft."""
    depth = []
    for i, p in enumerate(parents):
        p = int(p)
        if i == 0:
            if p != -1:
                raise ValueError("node 0 is the root and has parent -1")
            depth.append(0)
            continue
        if not 0 <= p < i:
            raise ValueError(f"node {i}: parent {p} is not an earlier node")
        depth.append(depth[p] + 1)
    return depth


def tree_mask(parents):
    """Ancestor-or-self mask uint8 [M, M]: mask[i][j] = 1 when j is i or one of its ancestors
    (reference spec_tree.py:101-104). A chain's mask is lower-triangular."""
    tree_depths(parents)
    m = len(parents)
    mask = np.zeros((m, m), dtype=np.uint8)
    for i in range(m):
        j = i
        while j != -1:
            mask[i, j] = 1
            j = int(parents[j])
    return mask


def accept_chain(targets, draft):
    """Number of leading draft tokens the target agrees with: draft[j] is accepted while
    targets[j] (the target's greedy token after cand[0..j]) equals it (reference
    spec_mega.py:106-110)."""
    acc = 0
    for t, d in zip(targets, draft):
        if int(t) != int(d):
            break
        acc += 1
    return acc


def accept_tree(cand, parents, targets):
    """Longest root-to-leaf path the target agrees with: from the root, step to the first child
    (in node order) whose token is the target's greedy token at the current node (reference
    spec_tree.py:109-118). Returns the node indices of the path, root first."""
    children = [[] for _ in cand]
    for i in range(1, len(cand)):
        children[int(parents[i])].append(i)
    path = [0]
    cur = 0
    while True:
        want = int(targets[cur])
        nxt = next((c for c in children[cur] if int(cand[c]) == want), None)
        if nxt is None:
            return path
        path.append(nxt)
        cur = nxt


def compaction_moves(path, pos):
    """(src, dst) cache slots that bring the accepted path's rows to slots pos..pos+L: node
    path[s] was written at slot pos+path[s] and belongs at pos+s (its RoPE already used position
    pos+s, its depth). Rows already in place are left out (reference spec_tree.py:125-128)."""
    src, dst = [], []
    for s in range(1, len(path)):
        if path[s] != s:
            src.append(pos + int(path[s]))
            dst.append(pos + s)
    return src, dst


class LookupDraft:
    """Prompt-lookup draft: find earlier occurrences of the context's last n tokens (n from
    max_ngram down to min_ngram, the most recent occurrence first) and propose what followed
    them. tree() merges up to `width` distinct continuations into a trie of at most
    max_nodes - 1 nodes below the root."""

    def __init__(self, max_ngram=3, min_ngram=1, width=2, depth=4, max_nodes=_lib.MAX_VERIFY):
        if not 1 <= min_ngram <= max_ngram:
            raise ValueError("need 1 <= min_ngram <= max_ngram")
        self.max_ngram, self.min_ngram = int(max_ngram), int(min_ngram)
        self.width, self.depth = int(width), int(depth)
        self.max_nodes = min(int(max_nodes), _lib.MAX_VERIFY)

    def reset(self):
        """Forget the indexed context (SpecDecoder.generate calls this at the start of a run)."""
        self._ctx, self._pos = [], {}

    def _index(self, ctx):
        """Positions of every n-gram (min_ngram <= n <= max_ngram) of ctx, oldest first, kept
        across calls and extended when ctx extends the indexed context (the loop's case: the
        whole indexed context must be a prefix of ctx, compared element by element)."""
        old = getattr(self, "_ctx", [])
        n0 = len(old)
        if not (n0 and len(ctx) >= n0 and ctx[:n0] == old):
            n0, self._pos = 0, {}
        for n in range(self.min_ngram, self.max_ngram + 1):
            for i in range(max(0, n0 - n + 1), len(ctx) - n + 1):
                self._pos.setdefault(tuple(ctx[i:i + n]), []).append(i)
        self._ctx = list(ctx)
        return self._pos

    def _continuations(self, context, k, limit):
        ctx = context if isinstance(context, list) else [int(t) for t in context]
        n_ctx = len(ctx)
        pos = self._index(ctx)
        found, seen = [], set()
        for n in range(min(self.max_ngram, n_ctx - 1), self.min_ngram - 1, -1):
            for start in reversed(pos.get(tuple(ctx[n_ctx - n:]), ())):
                if start >= n_ctx - n:          # the suffix itself
                    continue
                cont = tuple(ctx[start + n:start + n + k])
                if cont and cont not in seen:
                    seen.add(cont)
                    found.append(list(cont))
                    if len(found) >= limit:
                        return found
        return found

    def chain(self, context, feats, k):
        conts = self._continuations(context, k, 1)
        return conts[0] if conts else []

    def tree(self, context, feats):
        tokens, parents = [], []
        kids = {}                                    # (parent, token) -> node; -1 = root
        for cont in self._continuations(context, self.depth, self.width):
            par = -1
            for t in cont:
                node = kids.get((par, t))
                if node is None:
                    if len(tokens) >= self.max_nodes - 1:
                        break
                    tokens.append(t)
                    parents.append(par)
                    node = kids[(par, t)] = len(tokens) - 1
                par = node
        return tokens, parents


class SpecStats:
    def __init__(self):
        self.passes = 0
        self.tokens = 0
        self.nodes = 0
        self.seconds = 0.0

    @property
    def tokens_per_pass(self):
        return self.tokens / self.passes if self.passes else 0.0

    def __repr__(self):
        return (f"SpecStats(passes={self.passes}, tokens={self.tokens}, nodes={self.nodes}, "
                f"tokens_per_pass={self.tokens_per_pass:.2f}, seconds={self.seconds:.4f})")


class SpecDecoder:
    """Greedy speculative decoding of one sequence on a flint_amd Transformer.

    generate(prompt, max_new, mode="chain" | "tree") sets up the model's caches (like
    generate.generate), prefills the prompt, and returns (prompt + new tokens as a host int list,
    SpecStats). Generation stops after max_new tokens or at the first eos token (which is kept).
    """

    def __init__(self, model, draft=None, k=4):
        self.model = model
        self.draft = draft if draft is not None else LookupDraft()
        self.k = int(k)
        if not 0 <= self.k < _lib.MAX_VERIFY:
            raise ValueError(f"k must be in [0, {_lib.MAX_VERIFY - 1}]")
        dev = model.device
        nv = _lib.MAX_VERIFY
        # tokens | depth | amask staged in one pinned buffer, one copy per pass
        self._host = torch.zeros(2 * nv + nv * nv // 4, dtype=torch.int32, pin_memory=dev.type == "cuda")
        self._dev = torch.zeros_like(self._host, device=dev)
        self._tout = torch.empty(nv, dtype=torch.int32, device=dev)
        self._feat = torch.empty(nv, model.config.dim, dtype=torch.bfloat16, device=dev)

    def _verify(self, cand, parents, pos):
        m = len(cand)
        nv = _lib.MAX_VERIFY
        vocab = self.model.config.vocab_size
        if any(not 0 <= t < vocab for t in cand):
            raise ValueError(f"draft token outside [0, {vocab})")
        h = self._host.numpy()
        h[:m] = cand
        h[nv:nv + m] = tree_depths(parents)
        h[2 * nv:].view(np.uint8)[:m * m] = tree_mask(parents).reshape(-1)
        self._dev.copy_(self._host, non_blocking=True)
        if m == 1:
            # a lone root is one decode step (same cache slot, RoPE position, argmax and final-norm
            # feature as a verify of M = 1), and the decode kernel is the faster of the two
            self.model.decode_step(self._dev[:1], pos, token_out=self._tout[:1], feat=self._feat[0])
            return self._tout[:1].tolist(), self._feat[:1]
        amask = self._dev[2 * nv:].view(torch.uint8)[:m * m].view(m, m)
        tout, _, feat = self.model.verify(self._dev[:m], pos, depth=self._dev[nv:nv + m], amask=amask,
                                          logits=False, feat=self._feat[:m], tokens_out=self._tout[:m])
        return tout[:m].tolist(), feat

    @torch.no_grad()
    def generate(self, prompt, max_new, mode="chain", eos=None):
        if mode not in ("chain", "tree"):
            raise ValueError("mode is 'chain' or 'tree'")
        if hasattr(self.draft, "reset"):
            self.draft.reset()
        ids = [int(t) for t in (prompt.reshape(-1).tolist() if torch.is_tensor(prompt) else prompt)]
        if not ids:
            raise ValueError("empty prompt")
        model, nv = self.model, _lib.MAX_VERIFY
        T = len(ids)
        max_seq = T + int(max_new) + nv
        model.setup_caches(1, max_seq)
        feats = torch.empty(max_seq, model.config.dim, dtype=torch.bfloat16, device=model.device)
        stats = SpecStats()
        out = list(ids)
        if max_new <= 0:
            return out, stats
        if T > 1:
            prefill(model, torch.tensor(ids[:-1], dtype=torch.int32), 0)
        pos = T - 1
        # reference spec_mega.py:92-93: the last prompt token through the verify kernel
        tgt, vfeat = self._verify([ids[-1]], [-1], pos)
        feats[0:1].copy_(vfeat[:1])
        n_feat, pos, nxt = 1, pos + 1, tgt[0]
        new = 0
        t0 = time.perf_counter()
        while True:
            out.append(nxt)
            new += 1
            if new >= max_new or nxt == eos:
                break
            room = min(nv, max_seq - pos)
            context = out
            if mode == "chain":
                d = [int(t) for t in self.draft.chain(context, feats[:n_feat], min(self.k, room - 1))]
                d = d[:room - 1]
                cand = [nxt] + d
                parents = list(range(-1, len(d)))
            else:
                toks, pars = self.draft.tree(context, feats[:n_feat])
                toks, pars = [int(t) for t in toks][:room - 1], [int(p) for p in pars][:room - 1]
                cand = [nxt] + toks
                parents = [-1] + [p + 1 for p in pars]          # draft parents -> verify node indices
            tgt, vfeat = self._verify(cand, parents, pos)
            path = accept_tree(cand, parents, tgt)
            if mode == "tree":
                src, dst = compaction_moves(path, pos)
                if src:
                    model.kv_move(src, dst)
            if path[-1] == len(path) - 1:                      # a prefix of the nodes
                feats[n_feat:n_feat + len(path)].copy_(vfeat[:len(path)])
            else:
                idx = torch.tensor(path, device=model.device)
                feats[n_feat:n_feat + len(path)].copy_(vfeat.index_select(0, idx))
            n_feat += len(path)
            stats.passes += 1
            stats.nodes += len(cand)
            stop = False
            for node in path[1:]:
                out.append(int(cand[node]))
                new += 1
                if new >= max_new or cand[node] == eos:
                    stop = True
                    break
            if stop:
                break
            pos += len(path)
            nxt = tgt[path[-1]]
        if model.device.type == "cuda":
            torch.cuda.synchronize()
        stats.seconds = time.perf_counter() - t0
        stats.tokens = new
        return out, stats
