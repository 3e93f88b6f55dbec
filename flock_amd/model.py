"""Greedy decoding of a whole Qwen3 model on libflock_attn (kernels/model.ts).

``Model`` follows model.ts's engine: token ids -> embedding gather (embed.wgsl,
over the tied token_embd) -> the decoder layers -> output norm -> LM head ->
argmax (model.ts:227-346). ``step(ids)`` feeds ids (a prompt, or one token)
and returns the next id; ``generate(prompt, maxTokens, eos)`` is the greedy
loop of model.ts:572-590.

Where the reference records each step into a WebGPU command buffer, here the
one-token step is captured once into a HIP graph and replayed: the position,
the token the embedding reads (the previous step's argmax) and the log of
generated ids all live in device memory, so a token costs one graph launch
and no host round trip; the host reads the whole log at the end.
"""
from __future__ import annotations

import numpy as np

from ._lib import CacheFullError
from . import ops
from .decoder import DecoderConfig, DecoderLayer


class Model:
    def __init__(self, cfg: DecoderConfig, layer_weights: list, token_embd, output_norm,
                 vocab: int, max_generate: int = 4096):
        self.cfg, self.vocab = cfg, vocab
        hid = cfg.hidden
        self.layers = [DecoderLayer.create(cfg, w) for w in layer_weights]
        self.embd = ops.Q8Matrix.from_packed(token_embd, vocab, hid)  # tied: embed + LM head
        self.g_out = ops.DeviceBuffer.from_array(np.ascontiguousarray(output_norm, np.float32))
        B = ops.DeviceBuffer
        P = max(1, cfg.maxPrefill)
        self.ids = B(4 * P)
        self.x = B(4 * P * hid)               # embedding output (layer 0's input)
        self.normed = B(4 * hid)
        self.tok_val, self.tok_idx = B(4), B(4)
        self.head_ws = B(ops.lm_head_ws_bytes(vocab, hid))
        self.state = B(8)                     # {position + 1, log cursor} of the captured step
        self.max_generate = max_generate
        self.log = B(4 * max_generate)
        self.nKeys = 0
        self.graph = None
        self._stream = None

    # ------------------------------------------------------------- host steps
    def reset(self) -> None:
        self.nKeys = 0
        for layer in self.layers:
            layer.reset()

    def _head(self, src_row) -> None:
        ops.lm_head(src_row, self.g_out, self.cfg.eps, self.embd, self.normed, None,
                    self.tok_val, self.tok_idx, self.head_ws)

    def step(self, ids) -> int:
        """Feed ``ids`` at positions nKeys.. and return the greedy next id
        (model.ts:387-393), prefilling in chunks of maxPrefill."""
        ids = np.ascontiguousarray(ids, np.uint32).ravel()
        if ids.size == 0:
            raise ValueError("step needs at least one token id")
        if self.nKeys + ids.size > self.cfg.maxKeys:
            raise CacheFullError(-2, f"KV cache would exceed {self.cfg.maxKeys} keys "
                                     f"({self.nKeys} + {ids.size})")
        P = max(1, self.cfg.maxPrefill)
        hid = self.cfg.hidden
        for off in range(0, ids.size, P):
            chunk = ids[off:off + P]
            n = chunk.size
            self.ids.upload(chunk)
            ops.embed(self.embd, self.ids, n, self.x)
            src = self.x
            for layer in self.layers:
                if n == 1:
                    layer.encode(src=src)
                else:
                    layer.encodePrefill(n, src=src)
                src = layer.outputBuffer()
            self.nKeys += n
        self._head(ops.ptr(src) + (n - 1) * hid * 4)
        ops.sync()
        return int(self.tok_idx.download(1, np.uint32)[0])

    # --------------------------------------------------------- captured steps
    def _capture(self) -> None:
        """Record the one-token step: embed(tok_idx) -> layers (position from
        n_keys_dev) -> head -> log the token, n_keys_dev += 1."""
        self._stream = ops.Stream()
        ops.set_stream(self._stream)
        with ops.Graph() as g:
            ops.embed(self.embd, self.tok_idx, 1, self.x)
            src = self.x
            for layer in self.layers:
                layer.encode_dev(src, self.state)  # state[0] = position + 1
                src = layer.outputBufferDev()
            self._head(src)
            ops.advance(self.state, 1, self.tok_idx, self.log, self.max_generate)
        self.graph = g

    def generate(self, prompt, maxTokens: int, eos=()) -> list:
        """Greedy decode (model.ts:572-590): the prompt is one host step, each
        further token one replay of the captured step."""
        if maxTokens < 1:
            return []
        if maxTokens > self.max_generate + 1:
            raise ValueError(f"maxTokens {maxTokens} exceeds max_generate {self.max_generate} + 1")
        first = self.step(prompt)
        rest = maxTokens - 1
        if self.nKeys + rest > self.cfg.maxKeys:
            raise CacheFullError(-2, f"KV cache full at {self.cfg.maxKeys} keys")
        out = [first] + (self.replay(first, rest) if rest > 0 else [])
        eos = set(int(e) for e in eos)
        for i, t in enumerate(out):
            if t in eos:
                return out[:i]
        return out

    def replay(self, first: int, n: int, read: bool = True) -> list:
        """Feed ``first`` at position nKeys and decode n tokens by replaying
        the captured step n times (the first n - 1 outputs are fed back on
        the device). Returns the n ids (read=False: leave them in the device
        log and return [])."""
        if self.nKeys + n > self.cfg.maxKeys:
            raise CacheFullError(-2, f"KV cache full at {self.cfg.maxKeys} keys")
        if n > self.max_generate:
            raise ValueError(f"{n} tokens exceed max_generate {self.max_generate}")
        if self.graph is None:
            self._capture()
        ops.set_stream(self._stream)
        self.state.upload(np.array([self.nKeys + 1, 0], np.uint32))
        self.tok_idx.upload(np.array([first], np.uint32))
        for _ in range(n):
            self.graph.launch()
        ops.sync()
        out = [int(t) for t in self.log.download(n, np.uint32)] if read else []
        self.nKeys += n
        for layer in self.layers:
            layer.nKeys = self.nKeys
        ops.set_stream(None)
        return out

    def free(self) -> None:
        if self.graph is not None:
            self.graph.free()
        if self._stream is not None:
            self._stream.free()
        for layer in self.layers:
            layer.free()
