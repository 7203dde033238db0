"""Token-by-token generation with a KV cache (memory_pool_model/generate.py:23-65).

Like the reference, every position, prompt included, is one decode step of
the backbone with its memory reads (MemoryPool: libmpl.so).  The decode step
has static shapes (token batch [B], position as a device tensor), so it is
captured once in a HIP graph and replayed; the next input token (the prompt's
or the argmax of the step's logits) is chosen on the device, so a whole
generation is queued without a host round trip per token.  For greedy
decoding a second graph also holds that choice (mpl_decode_next_token: the
prompt feed or the argmax, the output write and the position advance), so a
step is one replay with no other launch.  The reference's
jitted step takes the parameters on every call; here a generate() call
re-captures the step when a parameter was replaced, or when one that the
step reads through a copy made before capture (the pool's sub-keys and
log-temperature, the attention's query/key/value weights) changed in place
since the capture (other weights updated in place are read live by the
graph).
"""

from __future__ import annotations

import time
from typing import Dict, Optional

import numpy as np
import torch

from .model import MemoryPoolLM, ModelConfig


class Generator:
    """generate.py:23-65.  ``graph=False`` runs the decode step eagerly.
    With a file-mode host pool (rows read from the pool's .npy files on host
    threads) the step is not capturable and runs eagerly whatever ``graph``
    says; a RAM-mode host pool (pinned table read by the GPU) captures."""

    def __init__(self, mcfg: ModelConfig, params, batch_size: int = 1, graph: bool = True, device="cuda"):
        self.mcfg, self.batch_size, self.device = mcfg, batch_size, torch.device(device)
        self.params = params["params"] if "params" in params else params
        self.model = MemoryPoolLM(mcfg, decode=True)
        self.cache = self.model.init_cache(batch_size, self.device)
        self.tok = torch.zeros(batch_size, dtype=torch.int64, device=self.device)
        self.pos = torch.zeros(1, dtype=torch.int64, device=self.device)
        # the greedy graph's token step: prompt, its length and the generated
        # tokens stay on the device ([B, max_len] each)
        L = mcfg.max_len
        self.prompt_buf = torch.zeros((batch_size, L), dtype=torch.int64, device=self.device)
        self.out_buf = torch.zeros((batch_size, L), dtype=torch.int64, device=self.device)
        self.plen = torch.zeros(1, dtype=torch.int64, device=self.device)
        self.done = torch.zeros(1, dtype=torch.int32, device=self.device)  # the kernel's count, left at 0
        self.logits = None
        self.graph = None
        self.graph_greedy = None
        self.logits_greedy = None
        self.x_rows = None
        self._captured_state = None
        self.use_graph = graph

    def _step(self, input_rows=None):
        # The step's products have one row per stream.  For such shapes
        # hipBLASLt picks one-workgroup tiles; rocBLAS (torch's "cublas"
        # backend on ROCm) ran the 64-stream step 20% faster.  The choice is
        # torch's process-wide setting, so it is restored after the step (a
        # captured step keeps the kernels it was captured with).
        prev = torch.backends.cuda.preferred_blas_library()
        torch.backends.cuda.preferred_blas_library("cublas")
        try:
            logits, _ = self.model.apply({"params": self.params}, self.tok[:, None], positions=self.pos,
                                         cache=self.cache, input_rows=input_rows)
        finally:
            torch.backends.cuda.preferred_blas_library(prev)
        return logits[:, 0]

    def _next_token(self, logits, embed_into=None):
        """generate.py:44-61 for greedy decoding on the device: the next prompt
        token or the argmax of ``logits`` into self.tok, generated tokens into
        self.out_buf, then the position advanced (mpl_decode_next_token).
        With ``embed_into`` ([B, d_model] fp32) it also writes the next step's
        input rows there (mpl_decode_next_token_embed)."""
        from . import _lib

        lg = logits.float().contiguous()
        B, V = lg.shape
        P = _lib.ptr
        head = (P(lg), B, V, P(self.prompt_buf), self.prompt_buf.shape[1], P(self.plen), P(self.pos), P(self.tok),
                P(self.out_buf), self.out_buf.shape[1], self.out_buf.shape[1], P(self.done))
        if embed_into is None:
            _lib.check(_lib.lib().mpl_decode_next_token(*head, _lib.stream_ptr(self.device)),
                       "mpl_decode_next_token")
        else:
            emb, pe = self.params["embed"]["embedding"], self.params["pos_embed"]
            _lib.check(_lib.lib().mpl_decode_next_token_embed(
                *head, P(emb), emb.shape[0], P(pe), pe.shape[0], emb.shape[1], P(embed_into),
                _lib.stream_ptr(self.device)), "mpl_decode_next_token_embed")

    def _rows_in_token_step(self) -> bool:
        """Whether the greedy graph's token step can write the next step's
        input rows (fp32 contiguous 16-byte-aligned tables of a width that is
        a multiple of 4, as the GPU decode step's own embedding launch)."""
        emb, pe = self.params["embed"]["embedding"], self.params["pos_embed"]
        return (emb.shape[1] % 4 == 0 and emb.shape[1] == pe.shape[1]
                and all(t.dtype == torch.float32 and t.is_contiguous() and t.data_ptr() % 16 == 0 and t.is_cuda
                        for t in (emb, pe)))

    def _reset_cache(self):
        for c in self.cache:
            for t in c.values():
                t.zero_()

    def _param_state(self):
        """What a captured step depends on besides its inputs: the storage of
        every parameter (the graph reads the weights where they were at
        capture), and the in-place version of the parameters it reads through
        copies made before capture: the pool's sub-keys and log-temperature
        (packed operand, clamped value) and the attention's query/key/value
        weights (one fused projection)."""
        flat = []

        def walk(t):
            if isinstance(t, dict):
                for k in sorted(t):
                    walk(t[k])
            elif isinstance(t, torch.Tensor):
                flat.append(t.data_ptr())

        walk(self.params)
        pool = self.params.get("pool", {})
        copied = [pool[k] for k in ("sub_keys", "log_temperature") if k in pool]
        copied += self.model.copied_parameters(self.params)
        # identity too: a tensor replaced by a new one at the same address has
        # its version counter back at 0.  The state holds the tensors, so no
        # other tensor can take their ids while it is kept.
        return tuple(flat), tuple((t, id(t), t.data_ptr(), t._version) for t in copied)

    @staticmethod
    def _same_state(a, b) -> bool:
        if a is None or b is None or a[0] != b[0] or len(a[1]) != len(b[1]):
            return False
        return all(x[0] is y[0] and x[1:] == y[1:] for x, y in zip(a[1], b[1]))

    def _host_pool_off_device(self) -> bool:
        """True when the memory layers read a host pool in file mode: its rows
        are staged through host threads after a device-to-host read of the
        distinct ids, which a captured graph cannot hold."""
        pool = self.model.pool
        if pool is None or not pool.host_pool:
            return False
        from . import host_pool as hp

        return not hp.get(pool.host_pool).on_device_path

    def _ensure_graph(self):
        if not self.use_graph:
            return
        if self._host_pool_off_device():
            self.graph = self.graph_greedy = None  # file-mode host pool: every step runs eagerly
            return
        state = self._param_state()
        if self.graph is not None and self._same_state(state, self._captured_state):
            return
        self.graph = self.graph_greedy = None  # parameters moved or the pool's keys changed: capture again
        # warm up on a side stream (key packing, temperature, workspaces)
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(2):
                self._step()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        pool = self.model.pool
        if pool is not None:
            pool.frozen_under_capture = True  # keys and temperature are fixed while the graph replays
        try:
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.logits = self._step()
            # the greedy step: the same decode step, then the token choice
            # (the position it advances is reset by every generate()).  Its
            # token step also writes the next step's input rows (x_rows), so
            # the step reads them instead of embedding its tokens;
            # generate() forms the first ones
            self.x_rows = None
            if self._rows_in_token_step():
                self.x_rows = torch.empty((self.batch_size, self.mcfg.d_model), dtype=torch.float32,
                                          device=self.device)
            self.graph_greedy = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph_greedy):
                self.logits_greedy = self._step(input_rows=self.x_rows)
                self._next_token(self.logits_greedy, embed_into=self.x_rows)
        finally:
            if pool is not None:
                pool.frozen_under_capture = False
        self._captured_state = state

    def generate(self, prompt, n_new: int, temperature: float = 0.0, seed: int = 0,
                 keep_logits: bool = True, sync_each_step: bool = False) -> Dict[str, object]:
        """prompt [B, P] int tokens; greedy when temperature == 0.  Returns
        tokens [B, n_new], the logits of every step [B, P+n_new-1, vocab] (if
        keep_logits) and per-step wall times (measured only with
        sync_each_step, as the reference does)."""
        if not isinstance(prompt, torch.Tensor):
            prompt = torch.as_tensor(np.asarray(prompt))
        prompt = prompt.to(device=self.device, dtype=torch.int64)
        B, P = prompt.shape
        if B != self.batch_size:
            raise ValueError(f"batch of {B} prompts for a generator built for {self.batch_size}")
        if P + n_new > self.mcfg.max_len:
            raise ValueError("prompt + n_new exceeds max_len")
        with torch.no_grad():
            return self._generate(prompt, n_new, temperature, seed, keep_logits, sync_each_step)

    def _generate(self, prompt, n_new, temperature, seed, keep_logits, sync_each_step):
        B, P = prompt.shape
        self._ensure_graph()
        self._reset_cache()
        if temperature <= 0 and self.graph_greedy is not None:
            return self._generate_greedy_graph(prompt, n_new, keep_logits, sync_each_step)
        gen = torch.Generator(device=self.device).manual_seed(int(seed)) if temperature > 0 else None
        out, logits_all, times = [], [], []
        self.tok.copy_(prompt[:, 0])
        for pos in range(P + n_new - 1):
            t0 = time.perf_counter()
            self.pos.fill_(pos)
            if self.graph is not None:
                self.graph.replay()
                logits = self.logits
            else:
                logits = self._step()
            if pos + 1 < P:
                nxt = prompt[:, pos + 1]
            elif temperature > 0:
                nxt = torch.multinomial(torch.softmax(logits / temperature, -1), 1, generator=gen)[:, 0]
            else:
                nxt = torch.argmax(logits, -1)
            if keep_logits:
                logits_all.append(logits.clone())
            if pos + 1 >= P:
                out.append(nxt.clone())
            self.tok.copy_(nxt)
            if sync_each_step:
                torch.cuda.synchronize(self.device)
                times.append(time.perf_counter() - t0)
        toks = torch.stack(out, 1) if out else torch.zeros((B, 0), dtype=torch.int64, device=self.device)
        return {"tokens": toks,
                "logits": torch.stack(logits_all, 1) if keep_logits else None,
                "step_seconds": np.array(times)}

    def _generate_greedy_graph(self, prompt, n_new, keep_logits, sync_each_step):
        """Greedy generation as replays of the greedy graph alone: prompt,
        position, input token and generated tokens live on the device."""
        B, P = prompt.shape
        self.prompt_buf[:, :P].copy_(prompt)
        self.plen.fill_(P)
        self.pos.fill_(0)
        self.tok.copy_(prompt[:, 0])
        if self.x_rows is not None:  # the first step's input rows; the token step writes the others
            from .model import decode_embed
            self.x_rows.copy_(decode_embed(self.params["embed"]["embedding"], self.params["pos_embed"], self.tok,
                                           self.pos))
        logits_all, times = [], []
        for _ in range(P + n_new - 1):
            t0 = time.perf_counter()
            self.graph_greedy.replay()
            if keep_logits:
                logits_all.append(self.logits_greedy.clone())
            if sync_each_step:
                torch.cuda.synchronize(self.device)
                times.append(time.perf_counter() - t0)
        toks = self.out_buf[:, :n_new].clone()
        return {"tokens": toks,
                "logits": torch.stack(logits_all, 1) if keep_logits else None,
                "step_seconds": np.array(times)}
