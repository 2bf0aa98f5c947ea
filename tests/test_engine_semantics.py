"""Engine-level semantics over the Backend boundary: context shifting, mirroring
context_shift_keeps_generating_and_is_consistent (crates/rie-core/tests/
model.rs:492-521) on the reference's tiny llama with F16 weights, a 32-token
window and batches of 8.

A shift keeps the first tokens, drops half of the rest and evaluates the
remainder again at earlier positions, so the backend's cache slots are
rewritten with the position moving backwards (the Backend contract,
model/mod.rs:303-320).  The same checks run over the oracle (CPU) and over the
HIP backend (GPU)."""
import numpy as np
import pytest
import torch

import rust_interference_engine_amd as R
from rust_interference_engine_amd import synth
from ggml_np import F16
from naive_model import max_rel_err

N_CTX, MAX_BATCH, BOS = 32, 8, 1


def _context_shift_checks(make_backend):
    prompt = [BOS, 17, 42, 5]
    # generation runs past the 32-token window
    e = R.Engine(make_backend())
    out, stop, _ = e.generate(prompt, 100, bos=BOS)
    assert len(out) == 100 and stop == "max_tokens"
    assert len(e.cached) <= N_CTX
    # without shifting it stops at the window
    e = R.Engine(make_backend())
    out, stop, _ = e.generate(prompt, 100, context_shift=False, bos=BOS)
    assert stop == "context_full" and len(e.cached) == N_CTX
    # after a shift the cache state equals a fresh evaluation of the kept tokens
    e = R.Engine(make_backend())
    toks = [BOS] + [3 + (i * 7) % 300 for i in range(31)]
    e.eval_tokens(toks)
    assert e.shift_context(4, bos=BOS)
    kept = toks[:4] + toks[4 + 14:]
    assert e.cached == kept
    shifted = e.logits().copy()
    fresh = R.Engine(make_backend())
    fresh.eval_tokens(kept)
    err = max_rel_err(shifted, fresh.logits())
    assert err < 1e-4, f"shifted vs fresh: {err}"
    # nothing left to drop: the shift declines and the cache is unchanged
    e = R.Engine(make_backend())
    e.eval_tokens([BOS, 9])
    assert not e.shift_context(1, bos=BOS) and e.cached == [BOS, 9]
    return err


def test_context_shift_on_the_oracle(oracle):
    img = synth.build(synth.tiny("llama", F16))
    model = oracle.Model(img)
    _context_shift_checks(lambda: oracle.Backend(model, N_CTX, MAX_BATCH, 0, n_threads=2))


@pytest.mark.gpu
def test_context_shift_on_the_gpu():
    assert torch.cuda.is_available(), "needs the MI355X"
    img = synth.build(synth.tiny("llama", F16))
    _context_shift_checks(lambda: R.HipBackend(img, n_ctx=N_CTX, max_batch=MAX_BATCH))
