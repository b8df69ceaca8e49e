"""The condU language model around the DSQG layers, with O(1)-per-token generation.

``CondMTransformer`` has the constructor, parameter names, initialisation and forward of
train/train_2048_condU.py:320-365 (token + position embeddings, DSQG blocks with the
interference pool every ``interference_interval`` layers, one full causal-attention block at
``full_attn_layer``, final LayerNorm, LM head tied to the embedding), so the reference's
checkpoints load with ``strict=True``.  The DSQG layers run on the HIP kernels
(``DSQGBlock``); embeddings, LayerNorms, projections and the full-attention layer are torch.

``generate`` replaces the reference's ``generate()`` (train/train_2048_condU.py:463-487), which
re-runs the whole model on the last ``seq_len`` tokens for every new token.  Here a prompt is
prefilled once (one forward that also loads every layer's cache: the DSQG blocks' K/V rings
and pool sums, the full-attention layer's K/V rows) and each new token costs one decode step
per layer.  While the sequence fits the position table (at most ``seq_len`` tokens), this is
the reference's computation; beyond it the reference slides its window, which shifts every
position embedding, so each further token is recomputed on the window exactly as the
reference does.  Sampling follows the reference: greedy below temperature 0.01, else
temperature-scaled nucleus (top-p) sampling.
"""

from __future__ import annotations

from typing import List, Optional, Sequence

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from .modules import FFN, DSQGBlock


class FullCausalAttention(nn.Module):
    """train/train_2048_condU.py:210-245: softmax attention over all earlier tokens, with the
    DSQG layers' output gate.  ``prefill`` / ``step`` keep its K/V rows in a preallocated
    cache for generation."""

    def __init__(self, embedding_dim: int, num_heads: int, dropout: float = 0.1):
        super().__init__()
        self.embedding_dim = embedding_dim
        self.num_heads = num_heads
        self.head_dim = embedding_dim // num_heads
        self.qkv_proj = nn.Linear(embedding_dim, 3 * embedding_dim, bias=True)
        self.out_proj = nn.Linear(embedding_dim, embedding_dim, bias=True)
        self.gate_proj = nn.Linear(embedding_dim, embedding_dim, bias=True)
        nn.init.constant_(self.gate_proj.bias, 0.0)
        self.dropout_p = dropout

    def _heads(self, qkv: Tensor, B: int, N: int):
        H, HD = self.num_heads, self.head_dim
        return [t.view(B, N, H, HD).permute(0, 2, 1, 3) for t in qkv.split(self.embedding_dim, -1)]

    def _finish(self, out: Tensor, x: Tensor) -> Tensor:
        gate = torch.sigmoid(self.gate_proj(x))
        return F.dropout(self.out_proj(out * gate), p=self.dropout_p, training=self.training)

    def forward(self, x: Tensor, cache: Optional["_KVCache"] = None) -> Tensor:
        B, N, E = x.shape
        q, k, v = self._heads(self.qkv_proj(x), B, N)
        if cache is not None:
            cache.k[:, :, :N] = k
            cache.v[:, :, :N] = v
            cache.pos.fill_(N)
        # 16-bit inputs are attended in fp32: it keeps 16-bit batched products with transposed
        # operands (the math path of scaled_dot_product_attention) out of the layer.
        up = (lambda t: t.float()) if q.dtype in (torch.float16, torch.bfloat16) else (lambda t: t)
        out = F.scaled_dot_product_attention(
            up(q), up(k), up(v), attn_mask=None,
            dropout_p=self.dropout_p if self.training else 0.0, is_causal=True).to(q.dtype)
        return self._finish(out.permute(0, 2, 1, 3).reshape(B, N, E), x)

    @torch.no_grad()
    def step(self, x_t: Tensor, cache: "_KVCache") -> Tensor:
        """One token per sequence at the cache's position (a device tensor, so the step has
        fixed shapes and can be captured in a HIP graph): its K/V row goes to that slot and
        the query attends every slot up to it, in fp32."""
        B, E = x_t.shape
        q, k, v = self._heads(self.qkv_proj(x_t).unsqueeze(1), B, 1)
        slot = cache.pos[:1]
        cache.k.index_copy_(2, slot, k)
        cache.v.index_copy_(2, slot, v)
        T = cache.k.shape[2]
        mask = (torch.arange(T, device=x_t.device) <= slot).view(1, 1, 1, T)
        out = F.scaled_dot_product_attention(q.float(), cache.k.float(), cache.v.float(),
                                             attn_mask=mask)
        cache.pos += 1
        return self._finish(out.to(x_t.dtype).reshape(B, E), x_t)


class _KVCache:
    """K/V rows [B, H, T, HD] of the full-attention layer and the next position (device
    tensor [B]; every sequence of the batch is at the same position)."""

    def __init__(self, B: int, H: int, T: int, HD: int, dtype, device):
        self.k = torch.zeros((B, H, T, HD), dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.pos = torch.zeros((B,), dtype=torch.int64, device=device)


class FullAttentionBlock(nn.Module):
    """train/train_2048_condU.py:304-315: pre-norm block around FullCausalAttention + FFN."""

    def __init__(self, embedding_dim: int, num_heads: int, ffn_dim: int, dropout: float = 0.1):
        super().__init__()
        self.norm1 = nn.LayerNorm(embedding_dim)
        self.norm2 = nn.LayerNorm(embedding_dim)
        self.attn = FullCausalAttention(embedding_dim, num_heads, dropout)
        self.ffn = FFN(embedding_dim, ffn_dim, dropout)

    def forward(self, x: Tensor, cache: Optional[_KVCache] = None) -> Tensor:
        x = x + self.attn(self.norm1(x), cache)
        return x + self.ffn(self.norm2(x))

    def new_cache(self, batch: int, max_len: int, device=None, dtype=None) -> _KVCache:
        w = self.attn.qkv_proj.weight
        return _KVCache(batch, self.attn.num_heads, max_len, self.attn.head_dim,
                        dtype or w.dtype, device or w.device)

    def prefill(self, x: Tensor, cache: _KVCache) -> Tensor:
        return self.forward(x, cache)

    @torch.no_grad()
    def step(self, x_t: Tensor, cache: _KVCache) -> Tensor:
        x_t = x_t + self.attn.step(self.norm1(x_t), cache)
        return x_t + self.ffn(self.norm2(x_t))


class CondMTransformer(nn.Module):
    """train/train_2048_condU.py:320-365 with the DSQG blocks on the HIP kernels.  ``offsets``
    (default: the 44-offset table) selects the DSQG layers' offset table."""

    def __init__(self, vocab_size: int, embedding_dim: int, num_layers: int, num_heads: int,
                 ffn_dim: int, seq_len: int, full_attn_layer: int = 5,
                 interference_interval: int = 3, dropout: float = 0.1,
                 offsets: Optional[Sequence[int]] = None):
        super().__init__()
        self.seq_len = seq_len
        self.embedding = nn.Embedding(vocab_size, embedding_dim)
        self.pos_embed = nn.Embedding(seq_len + 2, embedding_dim)
        self.drop = nn.Dropout(dropout)
        self.full_attn_layer = full_attn_layer
        blocks = []
        for i in range(num_layers):
            if i == full_attn_layer:
                blocks.append(FullAttentionBlock(embedding_dim, num_heads, ffn_dim, dropout))
            else:
                blocks.append(DSQGBlock(
                    embedding_dim, num_heads, ffn_dim, seq_len, dropout=dropout,
                    use_checkpoint=False,
                    interference=(i % interference_interval == interference_interval - 1),
                    offsets=offsets))
        self.blocks = nn.ModuleList(blocks)
        self.norm = nn.LayerNorm(embedding_dim)
        self.out = nn.Linear(embedding_dim, vocab_size, bias=False)
        self.out.weight = self.embedding.weight
        self._init_weights()

    def _init_weights(self) -> None:
        """train/train_2048_condU.py:346-357: N(0, 0.02) weights, zero biases, gate bias 0."""
        for m in self.modules():
            if isinstance(m, nn.Linear):
                nn.init.normal_(m.weight, 0, 0.02)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)
            elif isinstance(m, nn.Embedding):
                nn.init.normal_(m.weight, 0, 0.02)
        for m in self.modules():
            if hasattr(m, "gate_proj") and isinstance(m.gate_proj, nn.Linear):
                nn.init.constant_(m.gate_proj.bias, 0.0)

    def forward(self, idx: Tensor) -> Tensor:
        B, N = idx.shape
        pos = torch.arange(N, device=idx.device).unsqueeze(0)
        x = self.drop(self.embedding(idx) + self.pos_embed(pos))
        for block in self.blocks:
            x = block(x)
        return self.out(self.norm(x))

    def param_count(self) -> int:
        return sum(p.numel() for p in self.parameters())

    # ---- generation ------------------------------------------------------------------------

    def new_cache(self, batch: int) -> "GenerationCache":
        """Per-block caches (DSQG rings and pool sums, the full-attention K/V rows) and the
        position of the next token."""
        caches = [b.new_cache(batch, self.seq_len) if isinstance(b, FullAttentionBlock)
                  else b.new_cache(batch) for b in self.blocks]
        dev = self.embedding.weight.device
        return GenerationCache(caches, torch.zeros((batch,), dtype=torch.int64, device=dev))

    def prefill(self, idx: Tensor, cache: "GenerationCache") -> Tensor:
        """Logits [B, N, V] of a prompt idx [B, N] (N <= seq_len); loads every layer's cache."""
        B, N = idx.shape
        assert N <= self.seq_len, f"prompt of {N} tokens exceeds the position table ({self.seq_len})"
        pos = torch.arange(N, device=idx.device).unsqueeze(0)
        x = self.drop(self.embedding(idx) + self.pos_embed(pos))
        for block, c in zip(self.blocks, cache.blocks):
            x = block.prefill(x, c)
        cache.pos.fill_(N)
        cache.n = N
        return self.out(self.norm(x))

    @torch.no_grad()
    def step(self, idx_t: Tensor, cache: "GenerationCache") -> Tensor:
        """Logits [B, V] of one new token per sequence (idx_t [B]) at the cache's position.
        Shapes are fixed and positions live on the device, so a step can be captured in a HIP
        graph and replayed for every further token.  The position must stay inside the position
        table and the full-attention cache (checked on the host, from the cache's host-side
        count, before anything is launched)."""
        if not cache.n < self.seq_len:
            raise ValueError(f"position {cache.n} is past the position table ({self.seq_len} "
                             "tokens); continue with forward() on the last seq_len tokens")
        cache.n += 1
        x = self.embedding(idx_t) + self.pos_embed(cache.pos)
        for block, c in zip(self.blocks, cache.blocks):
            x = block.step(x, c)
        cache.pos += 1
        return self.out(self.norm(x))

    @torch.no_grad()
    def generate(self, idx: Tensor, max_new: int, temperature: float = 1.0, top_p: float = 0.9,
                 generator: Optional[torch.Generator] = None, use_graph: bool = True) -> Tensor:
        """Append ``max_new`` sampled tokens to idx [B, N]; returns [B, N + max_new].

        After the prefill, the first step runs eagerly and the next ones replay it from a HIP
        graph (``use_graph``); sampling stays outside the graph.
        """
        was_training = self.training
        self.eval()
        ids = idx
        cache = None
        logits = None
        graph = side = None
        tok_in = logits_out = None
        for _ in range(max_new):
            n = ids.shape[1]
            if n <= self.seq_len:
                if cache is None:
                    cache = self.new_cache(ids.shape[0])
                    logits = self.prefill(ids, cache)[:, -1]
                # else: the last token's logits came from the previous step
            else:  # past the position table: the reference's sliding-window recomputation
                logits = self.forward(ids[:, -self.seq_len:])[:, -1]
            nxt = _sample(logits.float(), temperature, top_p, generator)
            ids = torch.cat([ids, nxt.unsqueeze(1)], dim=1)
            if ids.shape[1] > self.seq_len:
                continue
            if not use_graph:
                logits = self.step(nxt, cache)
            elif graph is not None:
                tok_in.copy_(nxt)
                graph.replay()
                cache.n += 1  # the replayed step advanced the device positions
                logits = logits_out
            else:
                # The first step runs eagerly on the capture stream (warming up every kernel and
                # library handle there); the second is captured and then replayed, as is every
                # later one.
                cur = torch.cuda.current_stream(ids.device)
                if side is None:
                    side = torch.cuda.Stream(ids.device)
                side.wait_stream(cur)
                if tok_in is None:
                    tok_in = nxt.clone()
                    with torch.cuda.stream(side):
                        logits = self.step(tok_in, cache)
                else:
                    tok_in.copy_(nxt)
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, stream=side):
                        logits_out = self.step(tok_in, cache)  # counts this token on the host
                    graph.replay()
                    logits = logits_out
                cur.wait_stream(side)
        self.train(was_training)
        return ids


class GenerationCache:
    """The caches of one generation: ``blocks[i]`` for block i, ``pos`` the next position (on
    the device, read by the kernels) and ``n`` the same count on the host."""

    def __init__(self, blocks: List, pos: Tensor):
        self.blocks = blocks
        self.pos = pos
        self.n = 0


def _sample(logits: Tensor, temperature: float, top_p: float,
            generator: Optional[torch.Generator]) -> Tensor:
    """train/train_2048_condU.py:474-484, per row: argmax below temperature 0.01, else nucleus
    sampling over the smallest set of tokens whose probability reaches top_p."""
    if temperature <= 0.01:
        return logits.argmax(dim=-1)
    probs = F.softmax(logits / temperature, dim=-1)
    sorted_probs, sorted_idx = torch.sort(probs, dim=-1, descending=True)
    cum = torch.cumsum(sorted_probs, dim=-1)
    sorted_probs = sorted_probs.masked_fill(cum - sorted_probs > top_p, 0.0)
    sorted_probs = sorted_probs / sorted_probs.sum(dim=-1, keepdim=True)
    pick = torch.multinomial(sorted_probs, 1, generator=generator)
    return sorted_idx.gather(-1, pick).squeeze(-1)
