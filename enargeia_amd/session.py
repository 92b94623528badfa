"""The per-token driver over eg_decoder: the host side of the reference's Session
(src/runtime/session.ts:85-500) for this path.

``generate`` is Session.generate (session.ts:416-469): the prompt through the prefill and its
first token sampled from the last prompt position (runPrefill + sampleFromPrefill, :326-344,
:472-495), then one decode step per token (decodeStep, :347-375) until ``max_tokens`` tokens, a
stop token or a full context. Sampling parameters and the seed are the session's
(``SessionOptions.sampling`` / ``seed``, default GREEDY and 0x5eed, :123-125); the history the
repetition penalty reads and the mulberry32 draw source live on the device inside the decoder,
so each step costs one launch sequence (or one graph replay) and one 4-byte readback.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

from .kernels import GREEDY, SamplingParams
from .model import Decoder


@dataclass
class GenerateTiming:
    """GenerateTiming (session.ts:59-67)."""

    ttft_seconds: float
    prefill_seconds: float
    inter_token_seconds: list = field(default_factory=list)
    tokens_per_second: float = 0.0


@dataclass
class GenerateResult:
    tokens: list
    timing: GenerateTiming


class Session:
    """A decoder, its position in the context and its sampling state."""

    def __init__(self, decoder: Decoder, sampling: SamplingParams = GREEDY, seed: int = 0x5EED,
                 capture: bool = True):
        self.decoder = decoder
        self.max_context = decoder.model.cfg.max_context
        self.filled = 0
        decoder.set_sampling(sampling.temperature, sampling.top_p, sampling.repetition_penalty)
        decoder.seed(seed)
        if capture:
            decoder.capture()

    @property
    def remaining(self) -> int:
        return self.max_context - self.filled

    def set_sampling(self, sampling: SamplingParams) -> None:
        self.decoder.set_sampling(sampling.temperature, sampling.top_p, sampling.repetition_penalty)

    def generate(self, prompt, max_tokens: int, stop_tokens=()) -> GenerateResult:
        prompt = [int(t) for t in prompt]
        if len(prompt) > self.remaining:  # session.ts:327-331
            raise RangeError(f"prompt of {len(prompt)} exceeds the remaining context of {self.remaining}")
        stop = set(int(t) for t in stop_tokens)
        started = time.perf_counter()
        nxt = self.decoder.prefill(self.filled, prompt)
        ttft = time.perf_counter() - started
        self.filled += len(prompt)
        produced = [nxt]
        inter = []
        i = 1
        while i < max_tokens and nxt not in stop:
            if self.remaining <= 0:
                break
            t = time.perf_counter()
            nxt = self.decoder.step()
            inter.append(time.perf_counter() - t)
            self.filled += 1
            produced.append(nxt)
            i += 1
        mean = sum(inter) / len(inter) if inter else ttft
        return GenerateResult(produced, GenerateTiming(ttft, ttft, inter, 1.0 / mean if mean > 0 else 0.0))


class RangeError(IndexError):
    """The reference's RangeError (a prompt past the remaining context)."""
