"""Algebraic transformer language model on top of the MI355X kernels.

API-identical to the reference ``kernels.algebraic_model``
(SkyeGunasekaran/fastAlgebraicTransformer algebraic_model.py:26-302): the same
module classes, constructor arguments, parameter and buffer names (so
state_dicts are interchangeable) and factory functions. On CUDA (HIP) tensors
the norm, attention and SwiGLU run the libkat kernels; on CPU tensors the
modules use the reference's torch formulas (algebraic_model.py:37-39, 58-60,
112-136), as the reference does.
"""

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from .backward import attention_torch, rational_attention_packed
from .forward import compute_alibi_slopes, rational_attention_decode
from .fused_ops import (EPS, add_mean_error_norm, mean_error_norm, rational_softmax,
                        rational_swiglu_packed)


def _narrow(x: torch.Tensor) -> Optional[torch.dtype]:
    """The dtype a norm output feeding an autocast matmul is cast to before
    the matmul reads it: the autocast dtype for an fp32 CUDA stream under
    autocast, else None (keep x's dtype). The fused norm writes that dtype
    directly, with the cast's own rounding, so the matmul's input is the
    same bits and the separate cast pass (and its backward) disappears."""
    if x.is_cuda and x.dtype == torch.float32 and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return None


class KVCache:
    """Keys and values of one block for cached decoding: [batch, max_len,
    n_head, d_head] each (token-major, as the qkv projection lays them out),
    allocated on first use in the dtype the projection produces (bf16 under
    autocast)."""

    def __init__(self, max_len: int):
        self.max_len = max_len
        self.k: Optional[torch.Tensor] = None
        self.v: Optional[torch.Tensor] = None


class RationalMR(nn.Module):
    """Mean-error normalisation, y = x / (mean|x| + eps) * weight
    (reference algebraic_model.py:26-39)."""

    def __init__(self, d_model: int, eps: float = EPS):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d_model))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return mean_error_norm(x, self.weight, self.eps)


class RationalSwiGLU(nn.Module):
    """Gated FFN: w_out(gate * sigma(gate) * value) with [gate | value] from one
    projection (reference algebraic_model.py:42-62)."""

    def __init__(self, d_model: int, d_ffn: int, dropout: float = 0.0):
        super().__init__()
        self.w_gate_val = nn.Linear(d_model, 2 * d_ffn, bias=False)
        self.w_out = nn.Linear(d_ffn, d_model, bias=False)
        self.dropout = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # gate, value = w_gate_val(x).chunk(2, dim=-1), read in place from the
        # packed projection (its gradient is written as one buffer as well)
        return self.dropout(self.w_out(rational_swiglu_packed(self.w_gate_val(x))))


class AlgebraicAttention(nn.Module):
    """Causal multi-head rational attention with ALiBi
    (reference algebraic_model.py:65-136)."""

    def __init__(self, d_model: int, n_head: int, dropout: float = 0.1):
        super().__init__()
        assert d_model % n_head == 0
        self.d_model = d_model
        self.n_head = n_head
        self.d_head = d_model // n_head
        self.scale = 1.0 / math.sqrt(self.d_head)
        self.qkv = nn.Linear(d_model, 3 * d_model, bias=False)
        self.out = nn.Linear(d_model, d_model, bias=False)
        self.dropout = nn.Dropout(dropout)
        self.register_buffer("alibi_slopes", compute_alibi_slopes(n_head))

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, T, C = x.shape
        qkv = self.qkv(x).view(B, T, 3, self.n_head, self.d_head)
        if x.is_cuda:
            # causal, with the padding mask applied as the reference's CPU path
            # applies it (algebraic_model.py:129-131; its GPU path, :93-101,
            # drops the mask). The kernels read q, k, v in place from the
            # packed projection and write the output as [B, T, H, D], so no
            # layout copies are made.
            y = rational_attention_packed(qkv, self.alibi_slopes, self.scale, eps=EPS,
                                          key_mask=mask).view(B, T, C)
        else:
            q, k, v = qkv.permute(2, 0, 3, 1, 4)
            y = self._cpu_attention(q, k, v, mask).transpose(1, 2).contiguous().view(B, T, C)
        return self.dropout(self.out(y))

    def forward_cached(self, x: torch.Tensor, cache, pos0: int) -> torch.Tensor:
        """Causal attention of the tokens ``x`` at positions pos0.. over the
        cached keys before them, appending their keys and values to ``cache``
        = (k, v), each [B, max_len, H, D] (token-major, as the qkv projection
        lays them out). A prompt (pos0 == 0) runs the causal kernel on x; one
        new token runs the decode kernel over the cache (CUDA tensors). ``cache``
        is a KVCache."""
        B, T, C = x.shape
        qkv = self.qkv(x).view(B, T, 3, self.n_head, self.d_head)
        if cache.k is None:
            shape = (B, cache.max_len, self.n_head, self.d_head)
            cache.k = torch.empty(shape, dtype=qkv.dtype, device=qkv.device)
            cache.v = torch.empty(shape, dtype=qkv.dtype, device=qkv.device)
        assert pos0 + T <= cache.max_len, "KV cache is full"
        kc, vc = cache.k, cache.v
        kc[:, pos0:pos0 + T] = qkv[:, :, 1]
        vc[:, pos0:pos0 + T] = qkv[:, :, 2]
        if pos0 == 0:
            y = rational_attention_packed(qkv, self.alibi_slopes, self.scale, eps=EPS).view(B, T, C)
        else:
            assert T == 1, "after the prompt, tokens are decoded one at a time"
            n = pos0 + 1
            y, _ = rational_attention_decode(qkv[:, 0, 0], kc[:, :n].permute(0, 2, 1, 3),
                                             vc[:, :n].permute(0, 2, 1, 3), self.alibi_slopes,
                                             self.scale, eps=EPS)
            y = y.reshape(B, 1, C)
        return self.dropout(self.out(y))

    def decode_step(self, x: torch.Tensor, cache: KVCache, pos: torch.Tensor,
                    lengths: torch.Tensor) -> torch.Tensor:
        """One new token per batch row (x: [B, 1, C]) at the position held on the
        device in ``pos`` (int64 [1]), with ``lengths`` = pos + 1 (int32 [B]):
        its key and value go into the cache at ``pos`` and the decode kernel
        attends over the first ``lengths`` cached positions. No host-side
        position enters the computation, so the step can be captured in a
        HIP graph and replayed for every token."""
        B, T, C = x.shape
        qkv = self.qkv(x).view(B, 1, 3, self.n_head, self.d_head)
        cache.k.index_copy_(1, pos, qkv[:, :, 1])
        cache.v.index_copy_(1, pos, qkv[:, :, 2])
        y, _ = rational_attention_decode(qkv[:, 0, 0], cache.k.permute(0, 2, 1, 3),
                                         cache.v.permute(0, 2, 1, 3), self.alibi_slopes,
                                         self.scale, lengths=lengths, eps=EPS)
        return self.dropout(self.out(y.reshape(B, 1, C)))

    def _cpu_attention(self, q, k, v, mask):
        """Reference CPU path (algebraic_model.py:112-136): full score matrix,
        ALiBi, -1e4 causal and padding fill, rational softmax, P @ V."""
        return attention_torch(q, k, v, self.alibi_slopes, self.scale, mask, True, EPS)


class AlgebraicBlock(nn.Module):
    """Pre-norm residual block (reference algebraic_model.py:139-152)."""

    def __init__(self, d_model: int, n_head: int, d_ffn: int, dropout: float):
        super().__init__()
        self.attn = AlgebraicAttention(d_model, n_head, dropout)
        self.ffn = RationalSwiGLU(d_model, d_ffn, dropout)
        self.norm1 = RationalMR(d_model)
        self.norm2 = RationalMR(d_model)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        h, f = self.forward_pending(x, None, mask)
        return h + f

    def forward_pending(self, x: torch.Tensor, r: Optional[torch.Tensor],
                        mask: Optional[torch.Tensor] = None):
        """The block on the stream ``x + r`` (``r`` None: just ``x``), returning
        ``(h, f)`` with the block's output being ``h + f``. Each residual add
        is left to the norm that reads its result, which fuses the two
        (add_mean_error_norm), so the stream is read and written once per add."""
        if r is None:
            h0, n1 = x, self.norm1(x)
        else:
            h0, n1 = add_mean_error_norm(x, r, self.norm1.weight, self.norm1.eps, _narrow(x))
        h, n2 = add_mean_error_norm(h0, self.attn(n1, mask), self.norm2.weight, self.norm2.eps,
                                    _narrow(h0))
        return h, self.ffn(n2)

    def decode_pending(self, x: torch.Tensor, r: Optional[torch.Tensor], cache, pos: torch.Tensor,
                       lengths: torch.Tensor):
        """forward_pending for one new token (AlgebraicAttention.decode_step)."""
        if r is None:
            h0, n1 = x, self.norm1(x)
        else:
            h0, n1 = add_mean_error_norm(x, r, self.norm1.weight, self.norm1.eps, _narrow(x))
        h, n2 = add_mean_error_norm(h0, self.attn.decode_step(n1, cache, pos, lengths),
                                    self.norm2.weight, self.norm2.eps, _narrow(h0))
        return h, self.ffn(n2)

    def forward_pending_cached(self, x: torch.Tensor, r: Optional[torch.Tensor], cache, pos0: int):
        """forward_pending for tokens at positions pos0.. with the attention's
        keys and values kept in ``cache`` (AlgebraicAttention.forward_cached)."""
        if r is None:
            h0, n1 = x, self.norm1(x)
        else:
            h0, n1 = add_mean_error_norm(x, r, self.norm1.weight, self.norm1.eps, _narrow(x))
        h, n2 = add_mean_error_norm(h0, self.attn.forward_cached(n1, cache, pos0),
                                    self.norm2.weight, self.norm2.eps, _narrow(h0))
        return h, self.ffn(n2)


class AlgebraicTransformerLM(nn.Module):
    """Decoder-only LM with tied embedding/head (reference
    algebraic_model.py:155-265). Extra keyword arguments are accepted and
    ignored, as in the reference."""

    def __init__(
        self,
        vocab_size: int,
        d_model: int,
        n_head: int,
        n_layers: int,
        d_ffn: Optional[int] = None,
        block_size: int = 2048,
        dropout: float = 0.1,
        gradient_checkpointing: bool = False,
        **kwargs,
    ):
        super().__init__()
        d_ffn = int(d_model * 8 / 3) if d_ffn is None else d_ffn
        self.block_size = block_size
        self.gradient_checkpointing = gradient_checkpointing
        self.n_layers = n_layers
        self.embed = nn.Embedding(vocab_size, d_model)
        self.blocks = nn.ModuleList(
            [AlgebraicBlock(d_model, n_head, d_ffn, dropout) for _ in range(n_layers)])
        self.norm = RationalMR(d_model)
        self.head = nn.Linear(d_model, vocab_size, bias=False)
        self.embed.weight = self.head.weight  # weight tying
        self.apply(self._init_weights)

    def _init_weights(self, module):
        # N(0, 0.02) for Linear / Embedding weights, zero biases
        if isinstance(module, nn.Linear):
            std = 0.02
            if hasattr(module, "_scale_init"):
                std = 0.02 / math.sqrt(2 * self.n_layers)
            nn.init.normal_(module.weight, mean=0.0, std=std)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(
        self,
        input_ids: torch.Tensor,
        labels: Optional[torch.Tensor] = None,
        attention_mask: Optional[torch.Tensor] = None,
    ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        x = self.embed(input_ids)
        # the stream is carried as (x, r), x + r being the reference's x after
        # each block, so that every residual add fuses into the next norm
        r = None
        for block in self.blocks:
            if self.gradient_checkpointing and self.training:
                x, r = checkpoint(block.forward_pending, x, r, attention_mask, use_reentrant=False)
            else:
                x, r = block.forward_pending(x, r, attention_mask)
        if r is None:
            normed = self.norm(x)
        else:
            _, normed = add_mean_error_norm(x, r, self.norm.weight, self.norm.eps, _narrow(x))
        logits = self.head(normed)
        loss = None
        if labels is not None:
            # next-token loss: position t predicts token t+1 (algebraic_model.py
            # :229-236). The reference copies logits[..., :-1, :] into a new
            # tensor (and autograd scatters its gradient back); here the full
            # logits are used in place with the last position's target set to
            # the ignored index: the same terms and the same mean (up to the
            # summation order of the scalar loss), the same gradients.
            tgt = labels.new_full(labels.shape, -100)
            tgt[..., :-1] = labels[..., 1:]
            loss = F.cross_entropy(logits.reshape(-1, logits.size(-1)), tgt.reshape(-1),
                                   ignore_index=-100)
        return logits, loss

    def forward_cached(self, input_ids: torch.Tensor, caches, pos0: int) -> torch.Tensor:
        """Logits of the tokens ``input_ids`` at positions pos0.., attending to
        the keys and values of earlier positions held in ``caches`` (one
        KVCache per block, see new_kv_caches) and appending theirs. Equal to
        the corresponding rows of forward() on the whole sequence up to float
        rounding."""
        x = self.embed(input_ids)
        r = None
        for block, cache in zip(self.blocks, caches):
            x, r = block.forward_pending_cached(x, r, cache, pos0)
        normed = self.norm(x) if r is None else add_mean_error_norm(
            x, r, self.norm.weight, self.norm.eps, _narrow(x))[1]
        return self.head(normed)

    def decode_step(self, tokens: torch.Tensor, caches, pos: torch.Tensor,
                    lengths: torch.Tensor) -> torch.Tensor:
        """Logits [B, vocab] of one new token per row (tokens: [B, 1]) at the
        device-side position ``pos`` (int64 [1]; ``lengths`` = pos + 1, int32
        [B]) over filled ``caches``. Capturable in a HIP graph."""
        x = self.embed(tokens)
        r = None
        for block, cache in zip(self.blocks, caches):
            x, r = block.decode_pending(x, r, cache, pos, lengths)
        _, normed = add_mean_error_norm(x, r, self.norm.weight, self.norm.eps, _narrow(x))
        return self.head(normed)[:, -1, :]

    def new_kv_caches(self, max_len: int) -> list:
        """One KVCache per block, for up to ``max_len`` positions."""
        return [KVCache(max_len) for _ in self.blocks]

    @staticmethod
    def _sample(logits: torch.Tensor, temperature: float, top_k: Optional[int]) -> torch.Tensor:
        # algebraic_model.py:255-263
        if temperature != 1.0:
            logits = logits / temperature
        if top_k is not None:
            kth = torch.topk(logits, min(top_k, logits.size(-1)))[0][:, [-1]]
            logits[logits < kth] = float("-inf")
        return torch.multinomial(F.softmax(logits, dim=-1), num_samples=1)

    @torch.no_grad()
    def generate(self, idx: torch.Tensor, max_new_tokens: int, temperature: float = 1.0,
                 top_k: Optional[int] = None, use_cache: bool = True,
                 use_graph: bool = True) -> torch.Tensor:
        """Sample ``max_new_tokens`` tokens (reference algebraic_model.py:239-265).

        The reference re-runs the (cropped) prefix for every token. On CUDA
        tensors (``use_cache``) the prompt is run once into per-block key /
        value caches and each new token then costs one decode step; the logits
        are those of the full forward up to float rounding, and the sampling
        (temperature, top_k, multinomial) is the reference's. Once the context
        exceeds block_size the reference crops it, which changes every cached
        state, so from there on each token re-runs the cropped window as the
        reference does. ``use_cache=False`` (or CPU tensors) always does.
        With ``use_graph`` the one-token decode step is captured once in a HIP
        graph and replayed per token (under autocast it is captured with the
        autocast weight cache off, as graph capture requires)."""
        T0 = idx.size(1)
        cached = use_cache and idx.is_cuda and max_new_tokens > 0 and T0 <= self.block_size
        caches = None
        step = None
        for _ in range(max_new_tokens):
            n = idx.size(1)
            if cached and n <= self.block_size:
                if caches is None:
                    caches = self.new_kv_caches(min(T0 + max_new_tokens, self.block_size))
                    logits = self.forward_cached(idx, caches, 0)[:, -1, :]
                else:
                    if step is None:
                        step = _DecodeStep(self, caches, idx.size(0), idx.device, use_graph)
                    logits = step(idx[:, -1:], n - 1)
            else:
                ctx = idx if n <= self.block_size else idx[:, -self.block_size:]
                logits, _ = self.forward(ctx)
                logits = logits[:, -1, :]
            nxt = self._sample(logits, temperature, top_k)
            idx = torch.cat((idx, nxt), dim=1)
        return idx


class _DecodeStep:
    """The model's one-token decode step over fixed caches, run eagerly or as a
    captured HIP graph: the token ids, position and lengths live in static
    device buffers that are refilled before each replay."""

    def __init__(self, model, caches, batch: int, device, use_graph: bool):
        self.model, self.caches = model, caches
        self.tok = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self.pos = torch.zeros(1, dtype=torch.long, device=device)
        self.lengths = torch.ones(batch, dtype=torch.int32, device=device)
        self.use_graph = use_graph
        self.graph = None

    def _run(self):
        return self.model.decode_step(self.tok, self.caches, self.pos, self.lengths)

    def _capture(self):
        ac = torch.is_autocast_enabled()
        ac_dtype = torch.get_autocast_dtype("cuda") if ac else torch.float32
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            # the warm-up runs the step on the buffers already filled for the
            # first real step: it writes the cache row that step rewrites
            with torch.autocast("cuda", dtype=ac_dtype, enabled=ac, cache_enabled=False):
                self._run()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            with torch.autocast("cuda", dtype=ac_dtype, enabled=ac, cache_enabled=False):
                self.logits = self._run()
        self.graph = graph

    def __call__(self, tokens: torch.Tensor, pos: int) -> torch.Tensor:
        self.tok.copy_(tokens)
        self.pos.fill_(pos)
        self.lengths.fill_(pos + 1)
        if not self.use_graph:
            return self._run()
        if self.graph is None:
            self._capture()
        self.graph.replay()
        return self.logits


def create_small_model(vocab_size: int = 32000, **kwargs) -> AlgebraicTransformerLM:
    """d_model 768, 12 heads, 12 layers (~125M parameters)."""
    return AlgebraicTransformerLM(vocab_size=vocab_size, d_model=768, n_head=12, n_layers=12,
                                  **kwargs)


def create_medium_model(vocab_size: int = 32000, **kwargs) -> AlgebraicTransformerLM:
    """d_model 1024, 16 heads, 24 layers (~350M parameters)."""
    return AlgebraicTransformerLM(vocab_size=vocab_size, d_model=1024, n_head=16, n_layers=24,
                                  **kwargs)


def create_large_model(vocab_size: int = 32000, **kwargs) -> AlgebraicTransformerLM:
    """d_model 1536, 24 heads, 24 layers (~760M parameters)."""
    return AlgebraicTransformerLM(vocab_size=vocab_size, d_model=1536, n_head=24, n_layers=24,
                                  **kwargs)
