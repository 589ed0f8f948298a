"""GPU parity of speculative verify (fl_verify: M tokens through all layers in one launch, the
GEMMs on the matrix cores) against the CPU oracle's masked forward.

Reference semantics (kernels/verify_mega.cu:106-283, spec_mega.py:51-57, spec_tree.py:46-51,
101-104): token m sits at cache slot pos+m, takes RoPE position pos+depth[m] and attends to the
cache [0, pos) plus the new tokens j with amask[m][j]. Known-answer structure of the reference's
own test (bench/verify_mega_test.py:43-59): a causal chain verified in one pass equals M
sequential decode steps. Tolerance (tests/helpers.py check_rows): each row's max and mean |dlogit|,
and the mean over the rows, within twice the oracle's own floor (the larger of the configuration's
recorded floor and the distance of the oracle's second implementation on the same input), argmax
equal except where the oracle's top-2 margin is within the max bar.
"""
import pytest
import torch

from tests.helpers import (check_rows, compare_logits, fill_kv_random, log, make_pair,
                           oracle_pair)

pytestmark = pytest.mark.gpu

# The attention of a verify launch runs by tokens (a unit per query head and token group, every key
# in turn) or by key slices (a unit per query head and key slice on the matrix cores, partials
# merged), chosen by the launch's shape; FLINT_AMD_VERIFY_TOKEN_WORK at state creation forces one.
MODES = {"tokens": "1000000000", "slices": "0"}


@pytest.fixture(params=list(MODES))
def attn_mode(request, monkeypatch):
    monkeypatch.setenv("FLINT_AMD_VERIFY_TOKEN_WORK", MODES[request.param])
    return request.param


@pytest.mark.parametrize("name,pos,m", [("tiny", 0, 5), ("tiny", 77, 8), ("small", 130, 5),
                                        ("small", 200, 16), ("tiny", 300, 1), ("tiny", 3, 32),
                                        ("small", 60, 17), ("small", 250, 20), ("small", 90, 24),
                                        ("flint-3b-l1", 130, 28), ("flint-3b-l1", 300, 32),
                                        ("wide", 100, 8), ("wide", 40, 20)])  # D = 3072: 6 chunks a lane
def test_verify_chain_matches_oracle(dev, attn_mode, name, pos, m):
    args, sd, eng, orc = make_pair(name, seed=11)
    eng.setup_caches(1, 512)
    orc.setup_caches(eng.max_seq_length)
    fill_kv_random(eng, orc, pos, seed=pos + 3)
    g = torch.Generator().manual_seed(pos + m)
    toks = torch.randint(0, args.vocab_size, (m,), generator=g, dtype=torch.int32)
    tout, lg, feat = eng.verify(toks.to(dev), pos)
    eng.check()
    (alt, _), (lo, ho) = oracle_pair(orc, lambda: orc.forward(toks, pos))
    ties = check_rows(lg.cpu(), lo.float(), alt.float(), name, f"{name} {attn_mode} chain pos={pos} M={m}")
    assert ties <= max(1, m // 8)
    assert torch.equal(tout.cpu(), torch.argmax(lg.cpu(), dim=-1).int())
    assert float((feat.cpu().float() - ho.float()).abs().max()) <= 0.25
    # the M new K / V rows were appended at slots pos .. pos+M-1
    for l in range(args.n_layer):
        kd = (eng.k_cache[l, :, pos:pos + m].float().cpu() - orc.k_cache[l, :, pos:pos + m].float()).abs()
        vd = (eng.v_cache[l, :, pos:pos + m].float().cpu() - orc.v_cache[l, :, pos:pos + m].float()).abs()
        assert float(torch.maximum(kd, vd).max()) <= 0.25, l


def _random_tree(n, seed):
    """Parent list of an n-node tree in topological order: node i > 0 hangs off a node before it."""
    g = torch.Generator().manual_seed(seed)
    return [-1] + [int(torch.randint(0, i, (1,), generator=g)) for i in range(1, n)]


@pytest.mark.parametrize("name,pos,parent", [
    ("small", 150, [-1, 0, 0, 1, 1, 2, 3, 5]),
    ("small", 180, _random_tree(24, 3)),
    ("flint-3b-l1", 220, _random_tree(32, 4))])
def test_verify_tree_matches_oracle(dev, attn_mode, name, pos, parent):
    """Draft trees (spec_tree.py:46-51) of 8, 24 and 32 nodes: depth = node depth, amask =
    ancestors + self. Widths above 16 run the GEMM phases in two passes of 16 token rows."""
    args, sd, eng, orc = make_pair(name, seed=12)
    eng.setup_caches(1, 512)
    orc.setup_caches(eng.max_seq_length)
    fill_kv_random(eng, orc, pos, seed=21)
    m = len(parent)
    depth = torch.zeros(m, dtype=torch.int32)
    amask = torch.zeros(m, m, dtype=torch.uint8)
    for i in range(m):
        j = i
        while j >= 0:
            amask[i, j] = 1
            j = parent[j]
        depth[i] = int(amask[i].sum()) - 1
    toks = torch.randint(0, args.vocab_size, (m,), generator=torch.Generator().manual_seed(5),
                         dtype=torch.int32)
    tout, lg, feat = eng.verify(toks.to(dev), pos, depth=depth.to(dev), amask=amask.to(dev))
    eng.check()
    alt, lo = oracle_pair(orc, lambda: orc.forward(toks, pos, depth=depth, amask=amask)[0].float())
    ties = check_rows(lg.cpu(), lo, alt, name, f"{name} {attn_mode} tree M={m}")
    assert ties <= max(1, m // 8)


@pytest.mark.parametrize("m", [6, 32])
def test_verify_chain_equals_sequential_decode(dev, m):
    """Reference bench/verify_mega_test.py:43-59: verify of a causal chain == M decode steps."""
    args, sd, eng, _ = make_pair("tiny", seed=13)
    eng.setup_caches(1, 256)
    pos = 40
    g = torch.Generator().manual_seed(9)
    prefix = torch.randint(0, args.vocab_size, (pos,), generator=g, dtype=torch.int32).to(dev)
    toks = torch.randint(0, args.vocab_size, (m,), generator=g, dtype=torch.int32).to(dev)
    from flint_amd.generate import prefill
    prefill(eng, prefix, 0)
    _, lg_v, _ = eng.verify(toks, pos)
    lg_v = lg_v.cpu()
    logits = torch.empty(args.vocab_size, dtype=torch.float32, device=dev)
    for i in range(m):
        eng.decode_step(toks[i:i + 1], pos + i, logits=logits)
        ok, d, within, same = compare_logits(logits.cpu(), lg_v[i], "tiny")
        log(f"chain step {i}: max|dlogit| verify vs decode {d:.3e} ({same:.1%} identical)")
        assert ok
    eng.check()


def test_verify_rejects_bad_arguments(dev):
    from flint_amd import _lib
    args, sd, eng, _ = make_pair("tiny", seed=1)
    eng.setup_caches(1, 64)
    toks = torch.zeros(33, dtype=torch.int32, device=dev)
    with pytest.raises(_lib.FlError) as e:
        eng.verify(toks, 0)
    assert e.value.code == -3
    with pytest.raises(_lib.FlError) as e:
        eng.verify(toks[:4], 62)
    assert e.value.code == -2
    # the verify tiles read the tiled copies: without them fl_verify refuses (FL_E_ARG), and the
    # decode entry points, which read the row layout, still run
    eng._cw.wgu_t = None
    with pytest.raises(_lib.FlError) as e:
        eng.verify(toks[:4], 0)
    assert e.value.code == -1
    out = torch.empty(1, dtype=torch.int32, device=dev)
    eng.decode_step(toks[:1], 0, token_out=out)
    eng.check()


@pytest.mark.parametrize("name,pos", [("small", 40), ("small", 300), ("flint-3b-l1", 700)])
def test_verify_rows_do_not_depend_on_width(dev, attn_mode, name, pos):
    """A chain's first rows are computed the same way whatever the width (the GEMM rows are
    independent, token m attends to the same keys, the attention mode and key slicing depend on
    the context and the head count, here forced to one mode): verify of the first
    five tokens equals rows 0..4 of verify of all eight bit for bit, and a repeated launch equals
    the first (no dependence on workgroup timing)."""
    args, sd, eng, orc = make_pair(name, seed=31)
    eng.setup_caches(1, 1024)
    orc.setup_caches(eng.max_seq_length)
    fill_kv_random(eng, orc, pos, seed=pos)
    g = torch.Generator().manual_seed(pos)
    toks = torch.randint(0, args.vocab_size, (8,), generator=g, dtype=torch.int32).to(dev)
    _, l8, f8 = eng.verify(toks, pos)
    l8, f8 = l8.clone(), f8.clone()
    _, l8b, _ = eng.verify(toks, pos)
    _, l5, f5 = eng.verify(toks[:5], pos)
    eng.check()
    assert torch.equal(l8, l8b)
    d = (l5.float() - l8[:5].float()).abs().max().item()
    log(f"{name} pos={pos}: rows 0..4 at width 5 vs 8: max|d|={d:.3e}")
    assert torch.equal(l5, l8[:5]) and torch.equal(f5, f8[:5])
