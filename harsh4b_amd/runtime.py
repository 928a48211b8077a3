"""The reference's runtime interface over the MI355X decode path.

`inference_runtime.py` of the reference repository drives every backend
through one small interface (`Runtime`, :79-122): `prefill(ids, max_tokens)
-> (logits, session)`, `decode(token, session) -> logits`, `sample(logits,
generated, temperature) -> token`, and the token loop `stream(...)` built on
them, which the web UI and `bench_latency.py` consume.  `LiteSparkRuntime`
(:166-191) is the CPU int4 backend behind it.  `HipLiteSparkRuntime` here is
the same backend on one gfx950 GPU: the model is `lightspark.LiteSparkQwen`,
logits stay on the device, and `sample` runs `sample_numpy`'s policy
(:144-163) in one `hq_sample_token` launch.

The tokenizer is any object with the surface of the reference's
`ChatTokenizer` (:46-76) that the loop uses: `.backend` (a
`tokenizers.Tokenizer`) and `.stop_ids`.
"""
from __future__ import annotations

import time
from contextlib import contextmanager

import numpy as np

MODEL_ID = "Qwen/Qwen3-4B"

# sample_numpy's defaults (inference_runtime.py:144)
RUNTIME_TOP_P = 0.9
RUNTIME_TOP_K = 50
RUNTIME_REPETITION_PENALTY = 1.15
GREEDY_TEMPERATURE = 0.01


class Runtime:
    """Token loop and status shared by the backends (inference_runtime.py:79-122)."""

    device = "hip"
    description = ""
    hardware = ""
    max_context = 2048

    def status(self) -> dict:
        return dict(model=MODEL_ID, device=self.device, runtime=self.device,
                    hardware=self.hardware, quant=self.description, ready=True,
                    vram_gb=round(self.memory_gib(), 2), max_context=self.max_context)

    def memory_gib(self) -> float:
        return 0.0

    def prefill(self, ids, max_tokens):
        raise NotImplementedError

    def decode(self, token, session):
        raise NotImplementedError

    def sample(self, logits, generated, temperature):
        raise NotImplementedError

    def stream(self, prompt_ids, max_tokens, temperature, stopped=lambda: False):
        """The request loop of inference_runtime.py:90-122: a fresh session,
        the first token sampled from the prompt's logits, then one decode and
        one sample per further token until a stop id, `max_tokens` tokens or
        `stopped()`; no forward runs after the last token.  Yields
        {"token": text, "done": False} for each non-empty text piece and a
        last {"done": True, "stats": {...}} with the reference's keys."""
        from tokenizers.decoders import DecodeStream
        if not prompt_ids or len(prompt_ids) + max_tokens > self.max_context:
            raise ValueError("Prompt and output exceed the runtime context budget")
        clock = _Clock()
        produced: list[int] = []
        pieces = DecodeStream(skip_special_tokens=True)
        if not stopped():
            with clock.phase("prefill"):
                logits, session = self.prefill(prompt_ids, max_tokens)
                token = self.sample(logits, produced, temperature)
            while not stopped() and token not in self.tokenizer.stop_ids:
                produced.append(token)
                piece = pieces.step(self.tokenizer.backend, token)
                if piece:
                    yield {"token": piece, "done": False}
                if len(produced) >= max_tokens or stopped():
                    break
                with clock.phase("decode"):
                    token = self.sample(self.decode(token, session), produced, temperature)
        yield {"done": True, "stats": clock.stats(len(produced), round(self.memory_gib(), 2), self.device)}


class _Clock:
    """Wall time of the prefill phase and of each decode+sample step."""

    def __init__(self):
        self.seconds = {"prefill": 0.0, "decode": 0.0}
        self.decode_steps = 0

    @contextmanager
    def phase(self, name):
        t0 = time.perf_counter()
        yield
        self.seconds[name] += time.perf_counter() - t0
        self.decode_steps += name == "decode"

    def stats(self, tokens, vram_gb, runtime):
        prefill, decode = self.seconds["prefill"], self.seconds["decode"]
        return {"tokens": tokens, "time": round(prefill + decode, 3), "prefill_time": round(prefill, 3),
                "decode_time": round(decode, 3), "decode_steps": self.decode_steps,
                "tok_per_sec": round(self.decode_steps / decode, 2) if decode else 0.0,
                "vram_gb": vram_gb, "runtime": runtime}


class HipLiteSparkRuntime(Runtime):
    """LiteSparkRuntime (inference_runtime.py:166-191) on one MI355X.

    `rng` supplies the sampler's uniform draws through `random_sample()`;
    the reference's `sample_numpy` draws from numpy's global RandomState via
    `np.random.choice`, which is the default here too (so `np.random.seed`
    reproduces the reference's tokens).
    """

    description = "MI355X · LiteSpark packed int4 HIP"

    def __init__(self, model, tokenizer, rng=None):
        import torch
        self.model, self.tokenizer = model, tokenizer
        self.rng = rng if rng is not None else np.random     # np.random.random_sample: the global RandomState
        self.hardware = torch.cuda.get_device_name(model.device)
        self._session = None    # the decode state of the last prefill/decode

    @classmethod
    def from_cache(cls, directory, norms, tokenizer, model_path=None, config=None, rng=None):
        """A runtime over the reference's int4 cache directory (see harsh4b_amd.cache)."""
        from .cache import load_litespark_cache
        return cls(load_litespark_cache(directory, norms, config=config, model_path=model_path), tokenizer, rng)

    def prefill(self, ids, max_tokens):
        """A fresh session holding the prompt; the prompt runs through the
        batched prefill (the same bits as the reference's token loop)."""
        state = self.model.new_state(len(ids) + max_tokens)
        self._session = state
        return self.model.prefill(ids, state), state

    def decode(self, token, session):
        self._session = session
        return self.model.forward_token(int(token), session)

    def sample(self, logits, generated, temperature):
        """sample_numpy (inference_runtime.py:144-163): penalty 1.15 on the
        generated ids, then argmax when temperature <= 0.01 (no draw), else
        temperature, top-k 50, top-p 0.9 and np.random.choice's draw.  (The
        argmax branch ranks NaN after every number, where numpy's argmax
        would pick the first NaN.)"""
        from .lightspark import sample_token
        if temperature <= GREEDY_TEMPERATURE:
            token = sample_token(logits, generated, RUNTIME_REPETITION_PENALTY, 1.0, 1, 1.0, 0.0)[0]
        else:
            u = float(self.rng.random_sample())
            token = sample_token(logits, generated, RUNTIME_REPETITION_PENALTY, float(temperature),
                                 RUNTIME_TOP_K, RUNTIME_TOP_P, u)[0]
        # the token's step has finished (its logits were read): its status
        # word says whether that step ran as specified
        if self._session is not None:
            self._session.check_status()
        return token

    def memory_gib(self):
        import torch
        return torch.cuda.memory_allocated(self.model.device) / 2**30


def create_runtime(cache_directory, norms, tokenizer, model_path=None, **options) -> HipLiteSparkRuntime:
    """create_runtime (inference_runtime.py:349-356) for this backend: the
    reference's int4 cache of a checkpoint, its norm weights, and a
    tokenizer object with `.backend` and `.stop_ids` (the reference's
    ChatTokenizer is one)."""
    return HipLiteSparkRuntime.from_cache(cache_directory, norms, tokenizer, model_path=model_path, **options)
