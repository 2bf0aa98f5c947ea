"""Engine-level loops over a Backend, mirroring crates/rie-core/src/engine.rs:
prefix-reusing ``eval_tokens`` (250-272), ``shift_context`` (363-381),
``eval_next`` (384-392), the greedy path of ``generate`` (420-530), ``bench``
(540-564) and greedy argmax (sampler.rs:199-209)."""
from __future__ import annotations

import time

import numpy as np

from .backend import RieError


def argmax(x: np.ndarray) -> int:
    """sampler.rs:199-209: first index of the strict maximum (NaN never wins)."""
    x = np.asarray(x, np.float32)
    v = np.where(np.isnan(x), -np.inf, x)
    return int(np.argmax(v))


class Engine:
    def __init__(self, backend):
        self.backend = backend
        self.cached: list[int] = []
        self._logits = np.zeros(backend.n_vocab, np.float32)

    def reset(self) -> None:
        self.cached.clear()

    def logits(self) -> np.ndarray:
        return self._logits

    def eval_tokens(self, tokens) -> int:
        tokens = [int(t) for t in tokens]
        if not tokens:
            raise RieError(-5, "empty prompt")
        if len(tokens) > self.backend.n_ctx():
            raise RieError(-5, f"prompt of {len(tokens)} tokens exceeds context window of {self.backend.n_ctx()}")
        common = 0
        for a, b in zip(self.cached, tokens):
            if a != b:
                break
            common += 1
        if common == len(tokens):
            common -= 1
        del self.cached[common:]
        nb = self.backend.max_batch()
        pos = common
        while pos < len(tokens):
            end = min(pos + nb, len(tokens))
            self.backend.forward(tokens[pos:end], pos, False, self._logits)
            self.cached.extend(tokens[pos:end])
            pos = end
        return common

    def shift_context(self, n_keep: int, bos: int | None = None) -> bool:
        """Engine::shift_context (crates/rie-core/src/engine.rs:366-382): keep the first n_keep cached tokens (at least a
        leading BOS), drop half of the rest, and evaluate the remainder again at its
        new positions (its K/V carry the RoPE of the old ones); the kept prefix is
        reused.  False when nothing can be dropped."""
        n = len(self.cached)
        lead_bos = int(bos is not None and n > 0 and self.cached[0] == bos)
        keep = min(max(n_keep, lead_bos), n)
        discard = (n - keep) // 2
        if discard == 0:
            return False
        toks = self.cached[:keep] + self.cached[keep + discard:]
        del self.cached[keep:]
        self.eval_tokens(toks)
        return True

    def generate(self, tokens, max_tokens: int, context_shift: bool = True, n_keep: int = 0, bos: int | None = None,
                 stop_ids=()):
        """The greedy path of Engine::generate_hooked (crates/rie-core/src/engine.rs:420-537) without text handling: each
        step takes the argmax of the logits and counts it; a stop id ends the run
        unevaluated, a full window is shifted (or ends the run when shifting is off
        or frees nothing), and otherwise the token is evaluated.  Returns the tokens
        produced, the stop reason ("max_tokens", "end_of_sequence" or
        "context_full") and the number of prompt tokens reused from the cache."""
        reused = self.eval_tokens(tokens)
        out, stop = [], "max_tokens"
        while len(out) < max_tokens:
            tok = argmax(self._logits)
            out.append(tok)
            if tok in stop_ids:
                stop = "end_of_sequence"
                break
            if len(self.cached) >= self.backend.n_ctx() and (not context_shift or not self.shift_context(n_keep, bos)):
                stop = "context_full"
                break
            self.eval_next(tok)
        return out, stop, reused

    def eval_next(self, token: int) -> None:
        pos = len(self.cached)
        if pos >= self.backend.n_ctx():
            raise RieError(-5, "context window full")
        self.backend.forward([token], pos, False, self._logits)
        self.cached.append(int(token))

    def bench(self, n_prompt: int, n_gen: int):
        """Engine::bench with host-side argmax over read-back logits."""
        nv = self.backend.n_vocab
        toks = [(i * 7919 + 13) % nv for i in range(max(n_prompt, 1))]
        self.reset()
        self.eval_tokens(toks[:min(len(toks), 8)])
        self.reset()
        t0 = time.perf_counter()
        self.eval_tokens(toks)
        pp = time.perf_counter() - t0
        t1 = time.perf_counter()
        tok = argmax(self._logits)
        for _ in range(n_gen):
            self.eval_next(tok)
            tok = argmax(self._logits)
        tg = time.perf_counter() - t1
        self.reset()
        return len(toks) / pp, (n_gen / tg if n_gen else 0.0)

    def greedy(self, prompt, n_gen: int):
        """Prompt in max_batch chunks, then n_gen greedy steps on the device.
        Returns the n_gen tokens fed to the model (the first is the prompt's argmax)."""
        prompt = [int(t) for t in prompt]
        nb = self.backend.max_batch()
        pos = 0
        nxt = 0
        while pos < len(prompt):
            end = min(pos + nb, len(prompt))
            nxt = self.backend.forward_argmax(prompt[pos:end], pos)
            pos = end
        self.cached = list(prompt)
        out = self.backend.generate_greedy(pos, n_gen)
        self.cached.extend(int(t) for t in out)
        return out
