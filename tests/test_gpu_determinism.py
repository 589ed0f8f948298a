"""Run-to-run determinism of the persistent kernels at the benchmark's size (40-layer flint-3b).

Every reduction in k_decode and k_verify has a fixed order (wave partials merged in wave order,
key slices in slice order, down-projection parts in part order), and every exchange between
workgroups either carries the phase's tag or sits behind a ready flag written after the data. So
the same launch on the same inputs must give bit-identical logits, whatever the timing of the
256 workgroups and whatever tag values the launches carry. A missing wait in a hand-off (a word
read before its producer wrote it, a partial read from the previous launch) shows up here as a
rare logit difference, which the tolerance-based parity tests could miss.

Each case is launched several times at the same position (the launch rewrites its own K/V slots
with the same values) and the logits compared bitwise; the launches run at different epochs, so
every tag differs between repeats.
"""
import pytest
import torch

from flint_amd.synth import ModelArgs, synth_weights

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

REPEATS = 20


@pytest.fixture(scope="module")
def model(dev):
    from flint_amd.model import Transformer
    args = ModelArgs.from_name("flint-3b")
    eng = Transformer.from_weights(args, synth_weights(args, 0, device="cuda"), "cuda")
    # the attention by KV group (off by default) from 4096 cached keys, so that the decode cases
    # cover all three attentions
    mp = pytest.MonkeyPatch()
    mp.setenv("FLINT_AMD_GQA_MIN", "4096")
    eng.setup_caches(1, 4200)
    mp.undo()
    g = torch.Generator(device="cuda").manual_seed(11)
    eng.k_cache.normal_(generator=g)
    eng.v_cache.normal_(generator=g)
    yield args, eng
    eng.close()


def _same(runs):
    ref = runs[0]
    return [i for i, r in enumerate(runs[1:], 1) if not torch.equal(r, ref)]


# 1 key slice per head; 5 (slice 0 merging in the O phase); 5 at a long context; by KV group
@pytest.mark.parametrize("pos", [200, 600, 4000, 4150])
def test_decode_repeats_bitwise(model, pos):
    args, eng = model
    tok = torch.tensor([1234], dtype=torch.int32, device="cuda")
    runs = []
    for _ in range(REPEATS):
        lg = torch.empty(args.vocab_size, dtype=torch.float32, device="cuda")
        eng.decode_step(tok, pos, logits=lg)
        runs.append(lg)
    eng.check()
    torch.cuda.synchronize()
    assert _same(runs) == [], f"decode at pos {pos}: repeats differ from the first"


def _tree(m, seed):
    g = torch.Generator().manual_seed(seed)
    parent = [-1] + [int(torch.randint(0, i, (1,), generator=g)) for i in range(1, m)]
    depth = [0] * m
    mask = torch.zeros(m, m, dtype=torch.uint8)
    for i in range(m):
        j = i
        while j >= 0:
            mask[i, j] = 1
            j = parent[j]
        depth[i] = 0 if parent[i] < 0 else depth[parent[i]] + 1
    return torch.tensor(depth, dtype=torch.int32), mask


# attention by tokens for the first three, by key slices for the last two
@pytest.mark.parametrize("m,tree,pos", [(8, False, 1024), (5, False, 600), (24, True, 1024),
                                        (24, True, 2048), (32, False, 3000)])
def test_verify_repeats_bitwise(model, m, tree, pos):
    args, eng = model
    g = torch.Generator(device="cuda").manual_seed(m)
    toks = torch.randint(0, args.vocab_size, (m,), generator=g, dtype=torch.int32, device="cuda")
    depth = amask = None
    if tree:
        depth, amask = _tree(m, m)
        depth, amask = depth.cuda(), amask.cuda()
    runs = []
    for _ in range(REPEATS):
        out, lg, feat = eng.verify(toks, pos, depth=depth, amask=amask)
        runs.append(torch.cat([lg.flatten(), feat.float().flatten(), out.float()]))
    eng.check()
    torch.cuda.synchronize()
    assert _same(runs) == [], f"verify M={m} tree={tree} at pos {pos}: repeats differ from the first"
