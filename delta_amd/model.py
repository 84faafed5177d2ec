"""gpt-fast style decoder whose attention runs through the ``mylib::*`` ops on gfx950.

Mirrors DELTA/Engine/DELTA/model.py: ``ModelArgs`` and the model-shape table
(20-97), the paged ``KVCache`` buffer ``[pages, 2, 16, Hkv, d]`` (99-127), the
per-layer binding of ``attn_decode`` to ``target_decode`` /
``target_decode_plan`` (last full layer before a non-full one) /
``target_subset_decode`` (146-196), and the block structure (330-532).  The
GEMMs stay torch ops (hipBLASLt on ROCm).  By default (``fused=True``) the
element-wise chains between them are HIP kernels: the residual add + RMSNorm
(``delta_add_rmsnorm``), ``silu(w1 x) * w3 x`` on one merged (transposed) ``w13_t`` GEMM
(``delta_silu_mul``) and the final argmax (``delta_argmax_rows``), so a captured
decode step is not dominated by a dozen tiny launches per layer.  ``fused=False``
runs the reference's op-by-op structure (same math, same roundings).

No checkpoints ship with this build: ``init_random_weights`` gives every
parameter seeded N(0, std) values of the named architecture.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import torch
import torch.nn as nn
from torch import Tensor
from torch.nn import functional as F

from . import kernels as K
from . import ops  # noqa: F401  (registers the mylib:: ops)


def find_multiple(n: int, k: int) -> int:
    return n if n % k == 0 else n + k - (n % k)


@dataclass
class ModelArgs:
    block_size: int = 2048
    vocab_size: int = 32000
    n_layer: int = 32
    n_head: int = 32
    dim: int = 4096
    intermediate_size: Optional[int] = None
    n_local_heads: int = -1
    head_dim: int = 64
    rope_base: float = 10000
    norm_eps: float = 1e-5
    scaling_factor: float = 1.0
    low_freq_factor: Optional[int] = None
    high_freq_factor: Optional[int] = None
    original_max_position_embeddings: Optional[int] = None
    qkv_bias: bool = False
    full_cache_layers: Optional[List[int]] = None
    subset_cache_ratio: float = 0.5
    subset_cache_size: int = 0
    L: int = 8

    def __post_init__(self):
        if self.n_local_heads == -1:
            self.n_local_heads = self.n_head
        if self.intermediate_size is None:
            self.intermediate_size = find_multiple(int(2 * (4 * self.dim) / 3), 256)
        self.head_dim = self.dim // self.n_head
        if self.full_cache_layers is None:
            self.full_cache_layers = []

    @classmethod
    def from_name(cls, name: str):
        if name in transformer_configs:
            return cls(**transformer_configs[name])
        hits = [c for c in transformer_configs if c.lower() in str(name).lower()]
        if not hits:
            raise ValueError(f"unknown model shape {name!r}")
        hits.sort(key=len, reverse=True)
        return cls(**transformer_configs[hits[0]])


# Architecture shapes used by the benchmarks and the reference's recipes (model.py:72-97).
transformer_configs = {
    "llama-3-8b": dict(block_size=8192, n_layer=32, n_head=32, n_local_heads=8, dim=4096,
                       intermediate_size=14336, vocab_size=128256, rope_base=500000),
    "llama-3.1-8b": dict(block_size=131072, n_layer=32, n_head=32, n_local_heads=8, dim=4096,
                         intermediate_size=14336, vocab_size=128256, rope_base=500000.0, scaling_factor=8,
                         high_freq_factor=4, low_freq_factor=1, original_max_position_embeddings=8192),
    "Qwen2.5-7b": dict(block_size=131072, n_layer=28, n_head=28, n_local_heads=4, dim=3584,
                       intermediate_size=18944, vocab_size=152064, rope_base=1000000.0, qkv_bias=True,
                       norm_eps=1e-6),
    "Qwen2.5-14b": dict(block_size=131072, n_layer=48, n_head=40, n_local_heads=8, dim=5120,
                        intermediate_size=13824, vocab_size=152064, rope_base=1000000.0, qkv_bias=True,
                        norm_eps=1e-6),
    "DeepSeek-R1-Distill-Qwen-1.5B": dict(block_size=131072, n_layer=28, n_head=12, n_local_heads=2, dim=1536,
                                          intermediate_size=8960, vocab_size=151936, rope_base=10000.0,
                                          qkv_bias=True, norm_eps=1e-6),
    "DeepSeek-R1-Distill-Qwen-7B": dict(block_size=131072, n_layer=28, n_head=28, n_local_heads=4, dim=3584,
                                        intermediate_size=18944, vocab_size=152064, rope_base=10000.0,
                                        qkv_bias=True, norm_eps=1e-6),
    "DeepSeek-R1-Distill-Llama-8B": dict(block_size=131072, n_layer=32, n_head=32, n_local_heads=8, dim=4096,
                                         intermediate_size=14336, vocab_size=128256, rope_base=500000.0,
                                         scaling_factor=8, high_freq_factor=4, low_freq_factor=1,
                                         original_max_position_embeddings=8192),
    # small shape for tests: head_dim 128, GQA group 2
    "tiny-test": dict(block_size=4096, n_layer=4, n_head=4, n_local_heads=2, dim=512, intermediate_size=1024,
                      vocab_size=1000, rope_base=10000.0),
}


class KVCache(nn.Module):
    """One layer's paged cache ``[num_pages, 2, page_size, n_heads, head_dim]``."""

    def __init__(self, max_num_pages, page_size, n_heads, head_dim, dtype=torch.bfloat16):
        super().__init__()
        self.register_buffer("kv_cache", torch.zeros((max_num_pages, 2, page_size, n_heads, head_dim),
                                                     dtype=dtype), persistent=False)

    def update_target(self, k, v, kv_append_indptr, kv_page_indices, kv_page_indptr, kv_page_lastlen):
        torch.ops.mylib.update_kv(k, v, kv_append_indptr, self.kv_cache, kv_page_indices, kv_page_indptr,
                                  kv_page_lastlen)
        return self.kv_cache


class Transformer(nn.Module):
    def __init__(self, config: ModelArgs) -> None:
        super().__init__()
        self.config = config
        self.tok_embeddings = nn.Embedding(config.vocab_size, config.dim)
        self.layers = nn.ModuleList(TransformerBlock(config) for _ in range(config.n_layer))
        self.norm = RMSNorm(config.dim, eps=config.norm_eps)
        self.output = nn.Linear(config.dim, config.vocab_size, bias=False)
        self.layer_roles: List[str] = []
        self.fused = True

    def setup_caches(self, num_pages: int, page_size: int, kv_cache_pool: Optional[int] = None):
        """Allocate per-layer caches and bind each layer's attention op (model.py:146-196).

        ``kv_cache_pool`` = n (benchmarks of shapes whose KV exceeds HBM only): n physical caches,
        layer i uses cache i % n.  Every layer still reads and appends its own pages at the real
        shape; the values are shared between the layers of a cache, so the outputs are not a
        model's."""
        cfg = self.config
        head_dim = cfg.dim // cfg.n_head
        dtype = self.output.weight.dtype if self.output.weight.dtype == torch.float16 else torch.bfloat16
        full = set(cfg.full_cache_layers or [])
        self.layer_roles = []
        pool = None
        if kv_cache_pool is not None:
            n = int(kv_cache_pool)
            if n < 1:
                raise ValueError("kv_cache_pool must be >= 1")
            pool = [KVCache(num_pages, page_size, cfg.n_local_heads, head_dim, dtype) for _ in range(min(n, cfg.n_layer))]
        for i, b in enumerate(self.layers):
            if full:
                use_full = i in full
                next_full = (i + 1) in full if (i + 1) < cfg.n_layer else True
            else:
                use_full = next_full = True
            b.attention.kv_cache = (pool[i % len(pool)] if pool is not None
                                    else KVCache(num_pages, page_size, cfg.n_local_heads, head_dim, dtype))
            if use_full:
                if next_full:
                    b.attention.attn_decode = torch.ops.mylib.target_decode
                    self.layer_roles.append("full")
                else:
                    b.attention.attn_decode = torch.ops.mylib.target_decode_plan
                    self.layer_roles.append("plan")
            else:
                b.attention.attn_decode = torch.ops.mylib.target_subset_decode
                self.layer_roles.append("subset")
            b.attention.rope = torch.ops.mylib.rope
            b.attention.role = self.layer_roles[-1]

    def forward(self, idx: Tensor, input_pos: Tensor, kv_append_indptr: Tensor, kv_page_indices: Tensor,
                kv_page_indptr: Tensor, kv_page_lastlen: Tensor) -> Tensor:
        logits = self.forward_logits(idx, input_pos, kv_append_indptr, kv_page_indices, kv_page_indptr,
                                     kv_page_lastlen)
        return self._finalize_logits(logits)

    def forward_logits(self, idx, input_pos, kv_append_indptr, kv_page_indices, kv_page_indptr, kv_page_lastlen):
        x = self.tok_embeddings(idx)
        if not self.fused:
            for layer in self.layers:
                x = layer(x, input_pos, kv_append_indptr, kv_page_indices, kv_page_indptr, kv_page_lastlen)
            return self.output(self.norm(x))
        # Residual stream carried as (x, pending): block i's output x + ffn is summed by the
        # next block's fused add + norm.
        pending = None
        for layer in self.layers:
            x, pending = layer.forward_fused(x, pending, input_pos, kv_append_indptr, kv_page_indices,
                                             kv_page_indptr, kv_page_lastlen)
        _, y = K.add_rmsnorm(x, pending, self.norm.weight, self.norm.eps)
        return dense(y, self.output)

    def _finalize_logits(self, logits: Tensor) -> Tensor:
        """argmax over the vocabulary on the HIP kernel; returns int64 [bsz, seqlen]."""
        bsz, seqlen, vocab = logits.shape
        flat = logits.reshape(bsz * seqlen, vocab)
        out = torch.empty(bsz * seqlen, dtype=torch.int64, device=logits.device)
        K.argmax_rows(flat, out)
        return out.view(bsz, seqlen)

    @classmethod
    def from_name(cls, name: str):
        return cls(ModelArgs.from_name(name))


# Decode projections go to delta_gemm_skinny where it beats hipBLASLt on MI355X inside the
# captured step: every shape at <= 8 token rows.  At 32 rows it wins standalone for weights up to
# ~48 MB but loses inside the step (6.36 vs 6.17-6.25 ms per config-3 step, same process): its
# blocks re-read the activation rows, which the previous kernel left spread over the 8 XCDs'
# L2s, so the weight-size rule is off (0) until that re-read is gone.
_SKINNY_ROWS_ANY = 8
_SKINNY_MAX_WEIGHT_BYTES = 0


def dense(x: Tensor, layer: nn.Linear) -> Tensor:
    """``layer(x)`` on the decode GEMM kernel when it is the faster one, else torch."""
    w = layer.weight
    if K.gemm_skinny_ok(x, w):
        rows = x.numel() // x.shape[-1]
        if rows <= _SKINNY_ROWS_ANY or w.numel() * w.element_size() <= _SKINNY_MAX_WEIGHT_BYTES:
            return K.gemm_skinny(x, w, layer.bias)
    return layer(x)


# Projections whose only consumer is the next fused add + RMSNorm (wo, w2) go to delta_gemm_rows32
# at 9-32 token rows: it stages x in LDS per block and splits K across the grid, handing the
# norm fp32 partials to sum (Llama-3-8B at 32 rows: wo 9.5 vs 14.0 us, w2 24.6 vs 32.8 on
# hipBLASLt).  wqkv and the merged w1|w3 stay on hipBLASLt there (no gain without a consumer
# that sums partials, the same time for w1|w3).
_ROWS32_MAX = 32


def dense_to_norm(x: Tensor, layer: nn.Linear):
    """``layer(x)`` for a consumer that is ``K.add_rmsnorm``: the output, or the fp32 partials
    ``[S, rows, N]`` of a split-K ``delta_gemm_rows32`` that the norm sums."""
    w = layer.weight
    rows = x.numel() // x.shape[-1]
    if rows > _SKINNY_ROWS_ANY and rows <= _ROWS32_MAX and K.gemm_skinny_ok(x, w) and w.shape[0] % 64 == 0:
        r = K.gemm_rows32(x, w, layer.bias)
        return r if r.dtype == torch.float32 else r.view(*x.shape[:-1], w.shape[0])
    return dense(x, layer)


class TransformerBlock(nn.Module):
    def __init__(self, config: ModelArgs) -> None:
        super().__init__()
        self.attention = Attention(config)
        self.feed_forward = FeedForward(config)
        self.ffn_norm = RMSNorm(config.dim, config.norm_eps)
        self.attention_norm = RMSNorm(config.dim, config.norm_eps)

    def forward(self, x, offsets, kv_append_indptr, kv_page_indices, kv_page_indptr, kv_page_lastlen):
        h = x + self.attention(self.attention_norm(x), offsets, kv_append_indptr, kv_page_indices,
                               kv_page_indptr, kv_page_lastlen)
        return h + self.feed_forward(self.ffn_norm(h))

    def forward_fused(self, x, pending, offsets, kv_append_indptr, kv_page_indices, kv_page_indptr,
                      kv_page_lastlen):
        """Same block as ``forward`` with the input ``x + pending`` left unsummed; returns
        ``(h, ffn_out)`` whose sum is the block output."""
        x, a_in = K.add_rmsnorm(x, pending, self.attention_norm.weight, self.attention_norm.eps)
        attn = self.attention(a_in, offsets, kv_append_indptr, kv_page_indices, kv_page_indptr, kv_page_lastlen,
                              fused=True)
        h, f_in = K.add_rmsnorm(x, attn, self.ffn_norm.weight, self.ffn_norm.eps)
        return h, self.feed_forward.forward_fused(f_in)


class Attention(nn.Module):
    def __init__(self, config: ModelArgs):
        super().__init__()
        assert config.dim % config.n_head == 0
        total_head_dim = (config.n_head + 2 * config.n_local_heads) * config.head_dim
        self.wqkv = nn.Linear(config.dim, total_head_dim, bias=config.qkv_bias)
        self.wo = nn.Linear(config.dim, config.dim, bias=False)
        self.kv_cache: Optional[KVCache] = None
        self.attn_decode = None
        self.role = "full"  # which attention op the layer is bound to: full / plan / subset
        self.rope = None
        self.n_head = config.n_head
        self.head_dim = config.head_dim
        self.n_local_heads = config.n_local_heads
        self.dim = config.n_head * config.head_dim
        # debug capture (tests): when a list, each call appends (q, o)
        self.record: Optional[list] = None
        self._register_load_state_dict_pre_hook(self._merge_wq_wk_wv)

    @staticmethod
    def _merge_wq_wk_wv(state_dict, prefix, *args):
        """Checkpoints with separate q/k/v projections (and biases) load into the merged
        ``wqkv`` in q, k, v row order (the reference's load hook, model.py:392-405)."""
        for kind in ("weight", "bias"):
            names = [f"{prefix}{w}.{kind}" for w in ("wq", "wk", "wv")]
            if names[0] in state_dict:
                state_dict[f"{prefix}wqkv.{kind}"] = torch.cat([state_dict.pop(n) for n in names])

    def forward(self, x, offsets, kv_append_indptr, kv_page_indices, kv_page_indptr, kv_page_lastlen,
                fused: bool = False):
        bsz, seqlen, _ = x.shape
        q_size = self.n_head * self.head_dim
        kv_size = self.n_local_heads * self.head_dim
        lin = dense if fused else (lambda t, layer: layer(t))
        q, k, v = lin(x, self.wqkv).split([q_size, kv_size, kv_size], dim=-1)
        q = q.view(bsz * seqlen, self.n_head, self.head_dim)
        k = k.view(bsz * seqlen, self.n_local_heads, self.head_dim)
        v = v.view(bsz * seqlen, self.n_local_heads, self.head_dim)
        be = ops.active_backend()
        if fused and be.decode_append_ok():
            # Decode step: mylib::rope + mylib::update_kv + the layer's attention op in one launch
            # (bit-identical to the three).
            y = be.attn_append(self.role, q, k, v, offsets, self.kv_cache.kv_cache, kv_page_indices,
                               kv_page_indptr)
            if self.record is not None:  # the recorded query is the rotated one
                q = K.rope(q, k, kv_append_indptr, offsets, **be.rope_params())[0]
        else:
            if fused:
                # mylib::rope + mylib::update_kv in one launch (bit-identical to the two ops)
                q = K.rope_append(q, k, v, kv_append_indptr, offsets, self.kv_cache.kv_cache, kv_page_indices,
                                  kv_page_indptr, kv_page_lastlen, **be.rope_params())
                kv_cache = self.kv_cache.kv_cache
            else:
                q, k = self.rope(q, k, kv_append_indptr, offsets)
                kv_cache = self.kv_cache.update_target(k, v, kv_append_indptr, kv_page_indices, kv_page_indptr,
                                                       kv_page_lastlen)
            y = self.attn_decode(q, kv_cache)
        if self.record is not None:
            self.record.append((q.detach().clone(), y.detach().clone()))
        y = y.contiguous().view(bsz, seqlen, self.dim)
        return dense_to_norm(y, self.wo) if fused else lin(y, self.wo)


class FeedForward(nn.Module):
    """SwiGLU FFN.  ``w1`` and ``w3`` live in one weight stored transposed, ``w13_t``
    ``[dim, 2 * inter]``, so the gate and up projections are one GEMM ``x @ w13_t``: at
    32-row decode batches hipBLASLt streams this layout at ~5.2 TB/s against ~4.4 TB/s for
    ``x @ w13.T``.  An engine set up for at most 32 rows per step re-lays it out row-major
    (``w13`` ``[2 * inter, dim]``, ``use_row_major_w13``): ``delta_gemm_skinny`` streams it faster
    still at <= 8 rows (Qwen2.5-7B, 4 rows: 41 vs 53 us) and ``delta_gemm_rows32_silu`` fuses the
    SiLU-mul into the GEMM at 9-32 rows.  Checkpoints with separate ``w1`` /
    ``w3`` (the reference's names, ``[inter, dim]`` each) are merged and transposed on load."""

    def __init__(self, config: ModelArgs) -> None:
        super().__init__()
        self.inter = config.intermediate_size
        self.w13_t = nn.Parameter(torch.empty(config.dim, 2 * config.intermediate_size))
        self.w2 = nn.Linear(config.intermediate_size, config.dim, bias=False)
        self._register_load_state_dict_pre_hook(self._merge_w1_w3)

    def _merge_w1_w3(self, state_dict, prefix, *args):
        """Separate ``w1`` / ``w3`` weights load into the merged gate|up parameter in whichever
        layout this module holds it (transposed ``w13_t`` or row-major ``w13``)."""
        if prefix + "w1.weight" in state_dict:
            w13 = torch.cat([state_dict.pop(prefix + "w1.weight"), state_dict.pop(prefix + "w3.weight")])
            if hasattr(self, "w13"):
                state_dict[prefix + "w13"] = w13
            else:
                state_dict[prefix + "w13_t"] = w13.t().contiguous()

    @torch.no_grad()
    def use_row_major_w13(self) -> None:
        """Store the merged gate|up weight row-major, ``w13`` ``[2 * inter, dim]`` (same values)."""
        if hasattr(self, "w13_t"):
            w = self.w13_t.data.t().contiguous()
            del self.w13_t
            self.w13 = nn.Parameter(w, requires_grad=False)

    def _gate_up(self, x: Tensor) -> Tensor:
        if hasattr(self, "w13"):
            if K.gemm_skinny_ok(x, self.w13) and x.numel() // x.shape[-1] <= _SKINNY_ROWS_ANY:
                return K.gemm_skinny(x, self.w13)
            return F.linear(x, self.w13)
        return torch.matmul(x, self.w13_t)

    def forward(self, x: Tensor) -> Tensor:
        g, u = self._gate_up(x).split(self.inter, dim=-1)
        return self.w2(F.silu(g) * u)

    def forward_fused(self, x: Tensor):
        """The block's FFN output for the next fused add + norm (maybe as fp32 partials)."""
        rows = x.numel() // x.shape[-1]
        if hasattr(self, "w13") and self.inter % 32 == 0 and K.gemm_skinny_ok(x, self.w13):
            # gate/up GEMM and SiLU-mul in one launch (same bits as the two)
            if rows <= _SKINNY_ROWS_ANY:
                return dense_to_norm(K.gemm_skinny_silu(x, self.w13), self.w2)
            if rows <= _ROWS32_MAX:
                return dense_to_norm(K.gemm_rows32_silu(x, self.w13), self.w2)
        return dense_to_norm(K.silu_mul(self._gate_up(x)), self.w2)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: Tensor) -> Tensor:
        xf = x.float()
        out = xf * torch.rsqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + self.eps)
        return out.type_as(x) * self.weight


@torch.no_grad()
def init_random_weights(model: Transformer, std: float = 0.02, seed: int = 0) -> Transformer:
    """Seeded N(0, std) linear/embedding weights, zero biases, unit norms (random-init checkpoint)."""
    gen = torch.Generator(device=next(model.parameters()).device)
    gen.manual_seed(seed)
    for name, p in model.named_parameters():
        if name.endswith("norm.weight") or ".attention_norm." in name or ".ffn_norm." in name:
            p.fill_(1.0)
        elif name.endswith(".bias"):
            p.zero_()
        else:
            p.normal_(0.0, std, generator=gen)
    return model


def build_random_model(name: str, device, dtype=torch.bfloat16, seed: int = 0, std: float = 0.02,
                       **overrides) -> Transformer:
    """Random-init model of the named shape, materialised directly on ``device``."""
    cfg = ModelArgs.from_name(name)
    for k, v in overrides.items():
        setattr(cfg, k, v)
    with torch.device("meta"):
        model = Transformer(cfg)
    model = model.to_empty(device=device).to(dtype)
    return init_random_weights(model, std=std, seed=seed).eval()
