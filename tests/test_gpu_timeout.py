"""The bounded-wait path of the persistent kernels, forced from the host.

Every inter-workgroup wait in k_decode / k_verify polls with a time bound and, once it is reached,
records FL_E_TIMEOUT and gives up, so a launch whose producer never arrives (a workgroup that is
not resident, a broken producer) still ends instead of hanging the GPU (the reference's grid
barriers have no such bound). These tests set the bound to one tick of the 100 MHz clock and make
workgroup 0 start with a wait on a word that is never written (fl_state_force_timeout), so that
wait gives up after its first 64 polls and every wait behind it follows: the launch must still end
normally, report FL_E_TIMEOUT through fl_state_check, and, after fl_state_reset with the default
bound restored, the same state must decode correctly again.
"""
import pytest
import torch

from tests.helpers import compare_logits, log, make_pair

pytestmark = pytest.mark.gpu

FL_E_TIMEOUT = -6


def _launch_code(run, eng):
    from flint_amd import _lib
    run()
    try:
        eng.check()
    except _lib.FlError as e:
        log(f"forced launch: {e}")
        return e.code
    return 0


@pytest.mark.parametrize("kind", ["decode", "verify"])
def test_forced_wait_timeout_then_recovery(dev, kind):
    args, sd, eng, orc = make_pair("small", seed=5)
    eng.setup_caches(1, 256)
    orc.setup_caches(eng.max_seq_length)
    tok = torch.tensor([17], dtype=torch.int32, device=dev)
    toks = torch.arange(3, 11, dtype=torch.int32, device=dev)
    eng.set_wait_limit(1)
    eng.force_timeout(True)
    if kind == "decode":
        code = _launch_code(lambda: eng.decode_step(tok, 0), eng)
    else:
        code = _launch_code(lambda: eng.verify(toks, 0), eng)
    assert code == FL_E_TIMEOUT
    eng.force_timeout(False)
    # the error stays until the state is reset
    from flint_amd import _lib
    with pytest.raises(_lib.FlError):
        eng.check()
    eng.set_wait_limit(0)
    eng.reset_state()
    eng.k_cache.zero_()
    eng.v_cache.zero_()
    logits = torch.empty(args.vocab_size, dtype=torch.float32, device=dev)
    for pos, t in enumerate((17, 250, 3)):
        out = eng.decode_step(torch.tensor([t], dtype=torch.int32, device=dev), pos, logits=logits)
        eng.check()
        lo, _ = orc.forward(torch.tensor([t]), pos)
        ok, d, within, same = compare_logits(logits.cpu(), lo[0].float(), "small")
        log(f"after recovery pos={pos}: max|dlogit|={d:.3e} argmax {int(out.item())}/{int(lo[0].argmax())}")
        assert ok
