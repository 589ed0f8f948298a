"""fl_sample_noalloc (the sampler with its scratch in a fixed device array instead of memory the
library allocates) against fl_sample, through the C ABI: the same tokens and bit-identical
probabilities on two calls in a row, the second with a smaller input (fewer rows, smaller
vocabulary, top-k on and off); sizes beyond the fixed scratch are rejected."""
import ctypes

import pytest
import torch

from flint_amd import _lib

pytestmark = pytest.mark.gpu


def _call(name, logits, rows, vocab, temp, top_k, seed, offset, tokens, probs):
    lib = _lib.load()
    fn = getattr(lib, name)
    return fn(_lib.ptr(logits), rows, vocab, ctypes.c_float(temp), top_k, ctypes.c_uint64(seed),
              ctypes.c_uint64(offset), None, _lib.ptr(tokens), _lib.ptr(probs), _lib.stream_ptr())


@pytest.mark.parametrize("first,second", [((3, 49152, 200), (2, 1000, 0)),
                                          ((17, 4096, 0), (1, 49152, 50))])
def test_sample_noalloc_matches_sample(dev, first, second):
    g = torch.Generator(device="cuda").manual_seed(11)
    for i, (rows, vocab, top_k) in enumerate((first, second)):
        lg = (torch.randn(rows, vocab, device="cuda", generator=g) * 2).to(torch.bfloat16).float()
        outs = {}
        for name in ("fl_sample", "fl_sample_noalloc"):
            tok = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
            pr = torch.empty(rows, vocab, dtype=torch.float32, device="cuda")
            _lib.check(name, _call(name, lg, rows, vocab, 0.8, top_k, 1234, 7 + i, tok, pr))
            torch.cuda.synchronize()
            outs[name] = (tok.cpu(), pr.cpu())
        ta, pa = outs["fl_sample"]
        tb, pb = outs["fl_sample_noalloc"]
        print(f"call {i}: rows {rows} vocab {vocab} top_k {top_k}: tokens {tb.tolist()[:6]}", flush=True)
        assert torch.equal(ta, tb)
        assert torch.equal(pa, pb)
        assert bool(((tb >= 0) & (tb < vocab)).all())


def test_sample_noalloc_rejects_oversized_input(dev):
    lg = torch.zeros(1, 8, dtype=torch.float32, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    rc = _call("fl_sample_noalloc", lg, 1, 65537, 1.0, 0, 0, 0, tok, None)
    assert rc == -1  # FL_E_ARG: vocab above the scratch's 65536


def test_sample_noalloc_in_a_captured_graph(dev):
    """The entry point is for callers that cannot allocate, code under HIP graph capture among
    them: captured once into a graph (after a first direct call, which looks the scratch address
    up), every replay over new logits written between replays gives the tokens and probabilities
    of a direct call on the same logits."""
    rows, vocab, top_k = 4, 49152, 200
    g = torch.Generator(device="cuda").manual_seed(5)
    lg = torch.empty(rows, vocab, dtype=torch.float32, device="cuda")
    tok = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    pr = torch.empty(rows, vocab, dtype=torch.float32, device="cuda")
    lg.copy_((torch.randn(rows, vocab, device="cuda", generator=g) * 2).to(torch.bfloat16).float())
    _lib.check("fl_sample_noalloc", _call("fl_sample_noalloc", lg, rows, vocab, 0.9, top_k, 77, 3, tok, pr))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _call("fl_sample_noalloc", lg, rows, vocab, 0.9, top_k, 77, 3, tok, pr)
    _lib.check("fl_sample_noalloc (captured)", rc)
    for i in range(4):
        lg.copy_((torch.randn(rows, vocab, device="cuda", generator=g) * 2).to(torch.bfloat16).float())
        tok.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        tg, pg = tok.cpu(), pr.cpu()
        td = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
        pd = torch.empty(rows, vocab, dtype=torch.float32, device="cuda")
        _lib.check("fl_sample_noalloc", _call("fl_sample_noalloc", lg, rows, vocab, 0.9, top_k, 77, 3, td, pd))
        torch.cuda.synchronize()
        print(f"replay {i}: tokens {tg.tolist()}", flush=True)
        assert torch.equal(tg, td.cpu()) and torch.equal(pg, pd.cpu())
        assert bool(((tg >= 0) & (tg < vocab)).all())
