"""The runtime adapter (harsh4b_amd.runtime) against the reference's Runtime
interface (inference_runtime.py:79-191 in the reference repository): the
request loop's control flow and stats on the CPU with a stub backend, the
sampler's draw against numpy's legacy np.random.choice, and on the GPU the
adapter over a model against an oracle-driven loop."""
import numpy as np
import pytest

from harsh4b_amd import runtime as rt

VOCAB = 512
STOP = 7


class Tok:
    """The part of the reference's ChatTokenizer the loop uses."""

    def __init__(self):
        from tokenizers import Tokenizer, models, pre_tokenizers
        vocab = {f"w{i}": i for i in range(VOCAB)}
        vocab["<|im_end|>"] = STOP
        del vocab[f"w{STOP}"]
        self.backend = Tokenizer(models.WordLevel(vocab, unk_token="w0"))
        self.backend.pre_tokenizer = pre_tokenizers.Whitespace()
        self.backend.add_special_tokens(["<|im_end|>"])
        self.stop_ids = {STOP}


def text_of(ids, tok):
    from tokenizers.decoders import DecodeStream
    d = DecodeStream(skip_special_tokens=True)
    return "".join(p for p in (d.step(tok.backend, t) for t in ids) if p)


class Stub(rt.Runtime):
    """Returns the scripted tokens; records the calls the loop makes."""

    def __init__(self, script):
        self.tokenizer, self.script, self.calls = Tok(), list(script), []

    def prefill(self, ids, max_tokens):
        self.calls.append(("prefill", len(ids), max_tokens))
        return "logits", "session"

    def decode(self, token, session):
        self.calls.append(("decode", token))
        return "logits"

    def sample(self, logits, generated, temperature):
        self.calls.append(("sample", list(generated)))
        return self.script.pop(0)


def run(r, *a, **kw):
    out = list(r.stream(*a, **kw))
    assert out[-1]["done"] and all(not o["done"] for o in out[:-1])
    return "".join(o["token"] for o in out[:-1]), out[-1]["stats"]


def test_stream_stops_at_stop_id_without_extra_forward():
    r = Stub([3, 4, 5, STOP, 9])
    text, stats = run(r, [1, 2], 10, 0.7)
    assert text == text_of([3, 4, 5], r.tokenizer)
    assert stats["tokens"] == 3 and stats["decode_steps"] == 3
    assert [c[0] for c in r.calls] == ["prefill", "sample"] + ["decode", "sample"] * 3
    # sample sees the tokens generated so far, the first one none
    assert r.calls[1] == ("sample", []) and r.calls[-1] == ("sample", [3, 4, 5])
    assert set(stats) == {"tokens", "time", "prefill_time", "decode_time", "decode_steps", "tok_per_sec",
                          "vram_gb", "runtime"}


def test_stream_max_tokens_and_stopped():
    r = Stub([3, 4, 5, 6])
    _, stats = run(r, [1], 2, 0.7)
    assert stats["tokens"] == 2 and stats["decode_steps"] == 1        # no forward after the last token
    flag = {"n": 0}

    def stopped():
        flag["n"] += 1
        return flag["n"] > 3
    r = Stub([3, 4, 5, 6, 7])
    _, stats = run(r, [1], 10, 0.7, stopped=stopped)
    assert stats["tokens"] < 4
    r = Stub([])
    _, stats = run(r, [1], 10, 0.7, stopped=lambda: True)
    assert stats["tokens"] == 0 and r.calls == []


def test_stream_context_budget():
    r = Stub([])
    with pytest.raises(ValueError, match="context budget"):
        list(r.stream([], 4, 0.7))
    with pytest.raises(ValueError, match="context budget"):
        list(r.stream([1] * 2000, 49, 0.7))
    assert r.status()["max_context"] == 2048 and r.status()["model"] == "Qwen/Qwen3-4B"


def test_legacy_choice_is_one_random_sample():
    # np.random.choice(ids, p=p) (sample_numpy's draw) takes one
    # random_sample() and searches the normalised float64 cdf (side right)
    for seed in range(200):
        rng = np.random.default_rng(seed)
        k = int(rng.integers(1, 60))
        p = rng.random(k).astype(np.float32)
        p[rng.random(k) < 0.3] = 0
        p[0] += np.float32(0.01)
        p /= p.sum(dtype=np.float32)
        ids = rng.permutation(10000)[:k]
        a = np.random.RandomState(seed).choice(ids, p=p)
        cdf = p.astype(np.float64).cumsum()
        cdf /= cdf[-1]
        u = np.random.RandomState(seed).random_sample()
        assert a == ids[np.searchsorted(cdf, u, side="right")]


def numpy_sample_argmax(logits, generated):
    """sample_numpy's temperature <= 0.01 branch (inference_runtime.py:145-151)."""
    values = np.array(logits, dtype=np.float32, copy=True)
    if generated:
        ids = np.array(sorted(set(generated)), dtype=np.int64)
        repeated = values[ids]
        values[ids] = np.where(repeated > 0, repeated / np.float32(1.15), repeated * np.float32(1.15))
    return int(values.argmax())


@pytest.mark.gpu
def test_hip_runtime_matches_oracle_loop(forward_golden):
    torch = pytest.importorskip("torch")
    import oracle
    from harsh4b_amd.synthetic import host_arrays
    from tests.test_gpu_step import golden_model
    print("\n[gpu] runtime adapter over the tiny model", flush=True)
    g = forward_golden
    model = golden_model(g)
    ref = oracle.OracleModel(g["config"], host_arrays(model))
    tok = Tok()
    prompt = [int(t) for t in g["tokens"][:5]]
    for temperature, seed in ((0.8, 3), (1.3, 4), (0.0, 0)):
        r = rt.HipLiteSparkRuntime(model, tok, rng=np.random.RandomState(seed))
        text, stats = run(r, prompt, 12, temperature)
        # the same loop on the oracle
        draws = np.random.RandomState(seed)
        rs = ref.new_state(len(prompt) + 12)
        for t in prompt:
            ref.forward_token(t, rs)
        want = []
        while True:
            if temperature <= 0.01:
                token = oracle.sample_token(rs.logits, want, 1.15, 1.0, 1, 1.0, 0.0)[0]
                assert token == numpy_sample_argmax(rs.logits, want)
            else:
                token = oracle.sample_token(rs.logits, want, 1.15, temperature, 50, 0.9, draws.random_sample())[0]
            if token == STOP:
                break
            want.append(token)
            if len(want) >= 12:
                break
            ref.forward_token(token, rs)
        assert text == text_of(want, tok), temperature
        assert stats["tokens"] == len(want) and stats["runtime"] == "hip"
    assert r.status()["ready"] and r.memory_gib() > 0
    torch.cuda.synchronize()
