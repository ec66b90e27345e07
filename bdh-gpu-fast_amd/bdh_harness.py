"""BDH model harness around the attention hot path (prefill, cached decode, train step).

A from-scratch model of the same computation as the reference's BDH
(bdh_baseline.py:109-151 semantics; the layer layout and cache flow of
bdh.py:947-1193), so the hot path can be measured where the model calls it:

* prefill tok/s (configs C2 and C5): one forward over (B, T) tokens;
* decode tok/s (config C3): ``generate`` with a packed KR/V cache, the new
  token's RoPE(x) written straight into its cache slot and attention read
  from capacity-strided cache views (no cast copies of the past); or, with
  ``cache_manager=True``, through ``bdh_cache.CacheManager`` driven by
  bdh.py's own call sequence (bdh.py:1000-1036);
* a training step (C4 at model level): forward, cross entropy, backward.

Per layer (x: (B, T, D), LayerNorm without affine, eps 1e-5):

    x_bthn  = relu(einsum("btd,hdn->bthn", x, encoder))        # (B, T, nh, N), as 2-D GEMMs
    yKV     = tril(RoPE(x_sparse) RoPE(x_sparse)^T, -1) x      # x_sparse = x_bthn as (B, nh, T, N)
    y_bthn  = relu(einsum("bhtd,hdn->bthn", LN(yKV), encoder_v))
    x       = LN(x + LN((x_bthn * y_bthn).view(B, T, nh*N) @ decoder))

then ``logits = x @ lm_head``.  The dense products run on torch (hipBLASLt);
RoPE and attention go through the ``kernels`` surface, ``impl="hip"`` for the
gfx950 kernels or ``"eager"`` for the reference's torch semantics.  Under
``torch.autocast(dtype=bfloat16)`` the GEMMs run in bf16 and LayerNorm in
fp32, as in the reference's AMP runs.
"""

from __future__ import annotations

import dataclasses
from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

import kernels
from bdh_cache import CacheManager


@dataclasses.dataclass
class BDHConfig:
    """Model shape (bdh_baseline.py:11-18); N = mlp_internal_dim_multiplier * n_embd // n_head."""

    n_layer: int = 6
    n_embd: int = 256
    n_head: int = 4
    mlp_internal_dim_multiplier: int = 128
    vocab_size: int = 256

    @property
    def n_latent(self) -> int:
        return self.mlp_internal_dim_multiplier * self.n_embd // self.n_head


class KVCache:
    """Packed per-layer cache of RoPE(x) rows and V rows (the roles of bdh_cache.py:226-324).

    ``kr``: (L, B, nh, capacity, N) and ``v``: (L, B, 1, capacity, D) in the
    storage dtype.  A forward over T new tokens writes rows
    ``[seq_len, seq_len + T)`` of every layer, reads the past through
    capacity-strided views of rows ``[0, seq_len)``, and ``commit`` then
    advances ``seq_len``.
    """

    def __init__(self, cfg: BDHConfig, batch: int, capacity: int, dtype: torch.dtype, device):
        L, nh, N, D = cfg.n_layer, cfg.n_head, cfg.n_latent, cfg.n_embd
        self.capacity = int(capacity)
        self.kr = torch.empty(L, batch, nh, self.capacity, N, dtype=dtype, device=device)
        self.v = torch.empty(L, batch, 1, self.capacity, D, dtype=dtype, device=device)
        self.seq_len = 0

    @property
    def dtype(self) -> torch.dtype:
        return self.kr.dtype

    def slot(self, level: int, T: int):
        """Views of the rows the next T tokens occupy."""
        if self.seq_len + T > self.capacity:
            raise ValueError(f"KVCache: {self.seq_len} + {T} rows exceed capacity {self.capacity}")
        return self.kr[level].narrow(2, self.seq_len, T), self.v[level].narrow(2, self.seq_len, T)

    def past(self, level: int):
        return self.kr[level].narrow(2, 0, self.seq_len), self.v[level].narrow(2, 0, self.seq_len)

    def span(self, level: int, T: int):
        """Past and the next T rows together (rows ``[0, seq_len + T)``)."""
        n = self.seq_len + T
        return self.kr[level].narrow(2, 0, n), self.v[level].narrow(2, 0, n)

    def commit(self, T: int) -> None:
        self.seq_len += int(T)


def _ln(x: torch.Tensor) -> torch.Tensor:
    return F.layer_norm(x, (x.size(-1),), eps=1e-5)


def _ln_rows_ok(t: torch.Tensor) -> bool:
    """Shapes the HIP row LayerNorm takes: D = 64 * 2^k <= 1024, fp32 or bf16."""
    d = t.size(-1)
    return t.dtype in (torch.float32, torch.bfloat16) and d % 64 == 0 and d <= 1024 and (d // 64) & (d // 64 - 1) == 0


def _ln_fast(y: torch.Tensor, x: Optional[torch.Tensor] = None, dt: Optional[torch.dtype] = None,
             out_bf16: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``LN(y)`` (in ``dt``) or ``LN(x + LN(y))`` (in x's dtype) as one HIP pass: the
    LayerNorm of the reference's _ln / _residual_ln (bdh.py:565-574, 731-750), fp32
    arithmetic as under autocast.  ``out_bf16`` also receives the result in bf16."""
    if _ln_rows_ok(y) and (x is None or _ln_rows_ok(x)):
        return kernels.layer_norm_rows(y, x, out_dtype=x.dtype if x is not None else dt, out_bf16=out_bf16)
    if x is None:
        out = _ln(y.float())
        out = out.to(dt) if dt is not None else out
    else:
        out = _ln(x + _ln(y.float()))
    if out_bf16 is not None:
        out_bf16.copy_(out)
    return out


# The dense products are 2-D matrix products (hipBLASLt GEMMs) on contiguous
# operands: no einsum and no batched product, whose bf16 forms with
# transposed-view operands (einsum transposes inside; autograd's backward of
# a batched product does too) have faulted ROCm GPUs.
def _encode(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """relu(einsum("btd,hdn->bthn", x, w)) as one GEMM: (B*T, D) @ (D, nh*N) -> (B, T, nh, N)."""
    nh, D, N = w.shape
    wc = w.permute(1, 0, 2).reshape(D, nh * N)
    return F.relu(x.reshape(-1, D) @ wc).view(*x.shape[:-1], nh, N)


def _encode_heads(y: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """relu(einsum("bhtd,hdn->bthn", y, w)): one GEMM per head, (B*T, D) @ (D, N), stacked to (B, T, nh, N)."""
    B, nh, T, D = y.shape
    outs = [y[:, h].reshape(B * T, D) @ w[h] for h in range(nh)]
    return F.relu(torch.stack(outs, dim=1)).view(B, T, nh, w.size(2))


# Inference forms on the HIP path (no autograd, so no backward products):
def _compute_dtype(t: torch.Tensor) -> torch.dtype:
    return torch.get_autocast_dtype(t.device.type) if torch.is_autocast_enabled(t.device.type) else t.dtype


def _encode_relu_epilogue(x: torch.Tensor, wc: torch.Tensor, zero: torch.Tensor, nh: int) -> torch.Tensor:
    """The encoder GEMM with the ReLU applied in its epilogue (hipBLASLt): x (B, T, D) @
    wc (D, nh*N) with a zero bias -> (B, T, nh, N)."""
    D = x.size(-1)
    out = torch._addmm_activation(zero, x.reshape(-1, D).to(wc.dtype), wc)
    return out.view(*x.shape[:-1], nh, wc.size(1) // nh)


# Token rows of x_sparse from the streaming encoder are nh*N + _XS_PAD elements
# apart: the score pass reads one k range of many rows at a time, and rows a
# power of two apart (64 / 128 KB) put those reads on few memory channels.
# Measured per layer (same box): C2 score pass 377 -> 348 us, C5 1475 -> 1323
# us, the encoder 306 -> 314 / 546 -> 540 us, C5's gated product 757 -> 784
# us; forward C2 8.96 -> 8.76 ms, C5 29.47 -> 28.47 ms (pads of 64 and 256
# elements: C2 8.79 and 9.03 ms, C5 28.45 and 28.41 ms), the same logits.
_XS_PAD = 128


def _encode_fast(x: torch.Tensor, prep: dict, nh: int) -> torch.Tensor:
    """The encoder and its ReLU on the HIP forward: the library's streaming kernel
    (``kernels.relu_gemm``, one workgroup per head and 256 tokens) for bf16 with
    n_embd 256 or 512 when there are enough token blocks to fill the chip, into
    token rows padded by _XS_PAD elements; hipBLASLt's ReLU-epilogue GEMM
    otherwise (decode steps, short prompts)."""
    B, T, D = x.shape
    wt = prep["enc_t"]
    N = wt.size(1)
    if (wt.dtype == torch.bfloat16 and ((D == 256 and N % 64 == 0) or (D == 512 and N % 32 == 0))
            and (B * T + 255) // 256 * nh >= 128):
        xb = x.to(wt.dtype).contiguous()
        rows = torch.empty(B, T, nh * N + _XS_PAD, dtype=wt.dtype, device=x.device)
        out = rows.narrow(2, 0, nh * N).unflatten(2, (nh, N))
        return kernels.relu_gemm(xb.unsqueeze(1).expand(B, nh, T, D), wt, out=out)
    return _encode_relu_epilogue(x, prep["enc"], prep["zero"], nh)


def _gated_product(x_bthn: torch.Tensor, y_ln: torch.Tensor, w: torch.Tensor, wt=None) -> torch.Tensor:
    """x_bthn * relu(encoder_v GEMM), token-major (B, T, nh, N).

    bf16 (K a multiple of 32, N of 8, one head's y and wt under 4 GiB): one HIP
    kernel, the GEMM with the gated product as its epilogue (its output never
    reaches HBM).  Otherwise one
    batched GEMM (nh, B*T, D) @ (nh, D, N) on contiguous operands into
    head-major rows, then one HIP pass for the ReLU and the product."""
    B, T, nh, N = x_bthn.shape
    D = y_ln.size(-1)
    dt = _compute_dtype(x_bthn)
    fits = B * nh * T * D * 2 <= 2**32 and N * D * 2 <= 2**32  # the kernel's 32-bit DMA offsets
    if dt == torch.bfloat16 and x_bthn.dtype == torch.bfloat16 and D % 32 == 0 and N % 8 == 0 and fits:
        if wt is None:
            wt = w.transpose(1, 2).to(dt).contiguous()  # (nh, N, D)
        return kernels.gated_gemm(y_ln.to(dt).contiguous(), wt, x_bthn)
    a = y_ln.permute(1, 0, 2, 3).reshape(nh, B * T, D).to(dt)
    y = torch.bmm(a, w.to(dt))  # (nh, B*T, N)
    return kernels.relu_mul(x_bthn, y.view(nh, B, T, N).permute(1, 2, 0, 3))


def _chains_decoder(x_bthn: torch.Tensor, y_ln: torch.Tensor, dec: torch.Tensor) -> bool:
    """Whether ``kernels.gated_decoder`` takes the layer's gated product and
    decoder: bf16 operands, n_embd = 256 (its K and D), N a multiple of 32,
    more than 256 tokens (a decode step keeps the split-K decoder), one
    head's rows of encoder_v and of the decoder under 4 GiB."""
    B, T, nh, N = x_bthn.shape
    D = y_ln.size(-1)
    return (x_bthn.dtype == torch.bfloat16 and y_ln.dtype == torch.bfloat16 and dec.dtype == torch.bfloat16
            and D == 256 and dec.size(1) == 256 and N % 32 == 0 and B * T > 256 and N * D * 2 < 2**32)


def _follows(past: torch.Tensor, new: torch.Tensor) -> Optional[torch.Tensor]:
    """past||new as one view when ``new`` is the rows right after ``past`` in the
    same buffer (the reserved slot after the committed rows), else None."""
    if (past.untyped_storage().data_ptr() != new.untyped_storage().data_ptr() or past.stride() != new.stride()
            or past.dtype != new.dtype or past.shape[:-2] != new.shape[:-2] or past.size(-1) != new.size(-1)):
        return None
    if new.storage_offset() != past.storage_offset() + past.size(-2) * past.stride(-2):
        return None
    return past.as_strided((*past.shape[:-2], past.size(-2) + new.size(-2), past.size(-1)), past.stride(),
                           past.storage_offset())


class BDH(nn.Module):
    """BDH language model; parameter names and shapes follow bdh_baseline.py:80-102."""

    def __init__(self, cfg: BDHConfig):
        super().__init__()
        self.config = cfg
        nh, D, N, V = cfg.n_head, cfg.n_embd, cfg.n_latent, cfg.vocab_size
        self.decoder = nn.Parameter(torch.empty(nh * N, D).normal_(std=0.02))
        self.encoder = nn.Parameter(torch.empty(nh, D, N).normal_(std=0.02))
        self.encoder_v = nn.Parameter(torch.empty(nh, D, N).normal_(std=0.02))
        self.embed = nn.Embedding(V, D)
        nn.init.normal_(self.embed.weight, mean=0.0, std=0.02)
        self.lm_head = nn.Parameter(torch.empty(D, V).normal_(std=0.02))
        self.register_buffer("freqs", kernels.get_freqs(N), persistent=False)
        self._wcache: dict = {}

    def _prepared(self, dt: torch.dtype):
        """Inference layouts of the weights in the compute dtype, rebuilt when a weight changes:
        encoder as (D, nh*N) with a zero bias (ReLU-epilogue GEMM) and transposed to (nh, N, D)
        (streaming encoder kernel), encoder_v transposed to
        (nh, N, D) (gated GEMM), decoder (nh*N, D)."""
        key = tuple((p.data_ptr(), p._version) for p in (self.encoder, self.encoder_v, self.decoder))
        hit = self._wcache.get(dt)
        if hit is not None and hit[0] == key:
            return hit[1]
        nh, D, N = self.encoder.shape
        with torch.no_grad():
            prep = {
                "enc": self.encoder.permute(1, 0, 2).reshape(D, nh * N).to(dt).contiguous(),
                "enc_t": self.encoder.transpose(1, 2).to(dt).contiguous(),
                "zero": torch.zeros(nh * N, dtype=dt, device=self.encoder.device),
                "encv_t": self.encoder_v.transpose(1, 2).to(dt).contiguous(),
                "dec": self.decoder.to(dt).contiguous(),
            }
        self._wcache = {dt: (key, prep)}
        return prep

    # ----------------------------------------------------------- attention
    def _attention_managed(self, level, x_sparse, v_tok, cache: CacheManager, impl, cos_sin):
        """One layer against a ``CacheManager`` in bdh.py's order: reserve
        before get_past and RoPE into the slot when the storage dtype is the
        compute dtype and v matches it, else get_past, attention, append
        (bdh.py:1000-1036, 389-461)."""
        T = x_sparse.size(2)
        out_kr = None
        if not torch.is_grad_enabled() and cache.storage_matches_compute and v_tok.dtype == cache.storage_dtype:
            out_kr, dst_v = cache.reserve(level, T)
            past_kr, past_v = cache.get_past(level)
            dst_v.copy_(v_tok)
            v_tok = dst_v
        else:
            past_kr, past_v = cache.get_past(level)
        if past_kr is None and T > 1 and impl == "hip":
            # cold prefill: the fused kernel also leaves RoPE(x) for the cache
            qr = out_kr if out_kr is not None else torch.empty_like(x_sparse, memory_format=torch.contiguous_format)
            out = kernels.bdh_attn_rope(x_sparse, v_tok, self.freqs, 0, out_kr=qr, impl="hip")
        else:
            qr = kernels.bdh_rope_rotate(x_sparse, *cos_sin, out=out_kr, impl=impl)
            if past_kr is None:
                out = (x_sparse.new_zeros(x_sparse.size(0), x_sparse.size(1), 1, v_tok.size(-1)) if T == 1
                       else kernels.bdh_attn(qr, qr, v_tok, impl=impl))
            elif T == 1:
                out = kernels.bdh_attn_decode(qr, past_kr, past_v, impl=impl)
            else:
                S = past_kr.size(2)
                kr_all, v_all = _follows(past_kr, qr), _follows(past_v, v_tok)
                if kr_all is None or v_all is None:
                    kr_all = qr.new_empty(qr.size(0), qr.size(1), S + T, qr.size(3))
                    kr_all[:, :, :S].copy_(past_kr)
                    kr_all[:, :, S:].copy_(qr)
                    v_all = v_tok.new_empty(v_tok.size(0), 1, S + T, v_tok.size(3))
                    v_all[:, :, :S].copy_(past_v)
                    v_all[:, :, S:].copy_(v_tok)
                out = kernels.bdh_attn_past(kr_all[:, :, S:], kr_all, v_all, S, impl=impl)
        if out_kr is None:
            cache.append(level, qr, v_tok)
        return out

    def _attention(self, level, x_sparse, v_tok, rope_start, cache, impl, cos_sin):
        """RoPE + strict-tril attention of one layer (bdh.py:348-483 flow)."""
        T = x_sparse.size(2)
        if isinstance(cache, CacheManager):
            return self._attention_managed(level, x_sparse, v_tok, cache, impl, cos_sin)
        if cache is None:
            if impl == "hip":
                return kernels.bdh_attn_rope(x_sparse, v_tok, self.freqs, rope_start, impl="hip")
            qr = kernels.bdh_rope_rotate(x_sparse, *cos_sin, impl="eager")
            return kernels.bdh_attn(qr, qr, v_tok, impl="eager")
        S = cache.seq_len
        slot_kr, slot_v = cache.slot(level, T)
        if not (v_tok.data_ptr() == slot_v.data_ptr() and v_tok.shape == slot_v.shape and v_tok.stride() == slot_v.stride()):
            slot_v.copy_(v_tok)  # (the residual LayerNorm may have written the slot already)
        if impl == "hip" and S == 0 and T > 1:
            # cold prefill into an empty cache: RoPE(x) lands in the KR slot from the fused kernel
            return kernels.bdh_attn_rope(x_sparse, slot_v, self.freqs, 0, out_kr=slot_kr, impl="hip")
        qr = kernels.bdh_rope_rotate(x_sparse, *cos_sin, out=slot_kr, impl=impl)
        if T == 1:
            if S == 0:  # position 0 attends to nothing
                return x_sparse.new_zeros(x_sparse.size(0), x_sparse.size(1), 1, v_tok.size(-1))
            past_kr, past_v = cache.past(level)
            return kernels.bdh_attn_decode(qr, past_kr, past_v, impl=impl)
        kr_all, v_all = cache.span(level, T)
        return kernels.bdh_attn_past(kr_all[:, :, S:], kr_all, v_all, S, impl=impl)

    # ------------------------------------------------------------- forward
    def forward(
        self,
        idx: torch.Tensor,
        targets: Optional[torch.Tensor] = None,
        *,
        cache: Optional[KVCache | CacheManager] = None,
        impl: Optional[str] = None,
        last_only: bool = False,
    ):
        """Logits (B, T, V) (or (B, 1, V) with ``last_only``) and the loss when ``targets`` is given.

        With ``cache`` the tokens continue the cached sequence: RoPE positions
        start at ``cache.seq_len`` and every layer's RoPE(x) and V rows are
        stored in the cache, which is committed at the end.
        """
        impl = kernels.resolve_attn_impl(impl)
        cfg = self.config
        B, T = idx.shape
        nh, N = cfg.n_head, cfg.n_latent
        rope_start = cache.seq_len if cache is not None else 0
        need_table = impl != "hip" or (cache is not None and (cache.seq_len > 0 or T == 1))
        cos_sin = kernels.rope_cos_sin(T, rope_start, self.freqs) if need_table else None

        fast = impl == "hip" and not torch.is_grad_enabled()
        x = _ln(self.embed(idx))  # (B, T, D)
        prep = self._prepared(_compute_dtype(x)) if fast else None
        # Under bf16 compute the encoder and the attention's V take the fp32 residual
        # stream x rounded to bf16 (autocast's matmuls, bdh.py:396-413, 861-912).  From
        # layer 1 on the residual LayerNorm writes that copy (xb) beside x; into the KV
        # cache's V slot when the cache stores bf16, so a decode step makes neither a
        # cast nor a slot copy.  The bits are those of x.to(bf16).
        xb = None
        v_bf16 = fast and (cache is None or (isinstance(cache, KVCache) and cache.dtype == torch.bfloat16))
        for level in range(cfg.n_layer):
            if fast:
                x_bthn = _encode_fast(x if xb is None else xb, prep, nh)
            else:
                x_bthn = _encode(x, self.encoder)
            x_sparse = x_bthn.permute(0, 2, 1, 3)  # (B, nh, T, N) view
            v_tok = x.unsqueeze(1)
            if v_bf16 and x_sparse.dtype == torch.bfloat16 and v_tok.dtype == torch.float32:
                # rounded once, the score x V pass streams half the bytes
                if xb is not None:
                    # (with a cache: the V slot the residual LayerNorm wrote, as the slot's own view)
                    v_tok = cache.slot(level, T)[1] if cache is not None else xb.unsqueeze(1)
                elif cache is None:
                    v_tok = v_tok.to(torch.bfloat16)
            y_kv = self._attention(level, x_sparse, v_tok, rope_start, cache, impl, cos_sin)
            if fast:
                y_ln = _ln_fast(y_kv, dt=_compute_dtype(x_bthn))
                if _chains_decoder(x_bthn, y_ln, prep["dec"]):
                    # the gated product chained into the decoder: xy never stored
                    y_mlp = kernels.gated_decoder(y_ln.contiguous(), prep["encv_t"], x_bthn, prep["dec"])
                else:
                    xy = _gated_product(x_bthn, y_ln, self.encoder_v, prep["encv_t"])
                    if B * T <= 256 and xy.dtype == torch.bfloat16:
                        # few rows (decode): split-K GEMM instead of a few tiles down K = nh*N
                        y_mlp = kernels.small_gemm(xy.view(B * T, nh * N), prep["dec"]).view(B, T, -1)
                    else:
                        y_mlp = xy.view(B, T, nh * N) @ prep["dec"]
            else:
                xy = x_bthn * _encode_heads(_ln(y_kv), self.encoder_v)
                y_mlp = xy.view(B, T, nh * N) @ self.decoder
            if fast:
                xb = None
                if level + 1 < cfg.n_layer and x_bthn.dtype == torch.bfloat16 and x.dtype == torch.float32:
                    if v_bf16 and cache is not None:
                        xb = cache.slot(level + 1, T)[1][:, 0]  # (B, T, D) view of the next layer's V rows
                    else:
                        xb = torch.empty(B, T, x.size(-1), dtype=torch.bfloat16, device=x.device)
                x = _ln_fast(y_mlp, x, out_bf16=xb)
            else:
                x = _ln(x + _ln(y_mlp))
        if isinstance(cache, CacheManager):
            cache.commit()
        elif cache is not None:
            cache.commit(T)
        if last_only:
            x = x[:, -1:]
        logits = x @ self.lm_head
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.reshape(-1, logits.size(-1)).float(), targets.reshape(-1))
        return logits, loss

    # ------------------------------------------------------------ generate
    @staticmethod
    def sample(logits: torch.Tensor, temperature: float = 1.0, top_k: Optional[int] = None,
               generator: Optional[torch.Generator] = None) -> torch.Tensor:
        """One token per row from (B, V) fp32 logits (bdh.py:679-729): scale by
        1/temperature; with top_k, softmax over the k largest and draw among them."""
        if temperature != 1.0:
            logits = logits / temperature
        if top_k is not None and top_k < logits.size(-1):
            values, indices = torch.topk(logits, top_k, dim=-1)
            pick = torch.multinomial(torch.softmax(values, dim=-1), 1, generator=generator)
            return indices.gather(1, pick)
        return torch.multinomial(torch.softmax(logits, dim=-1), 1, generator=generator)

    @torch.no_grad()
    def generate(
        self,
        idx: torch.Tensor,
        max_new_tokens: int,
        temperature: float = 1.0,
        top_k: Optional[int] = None,
        *,
        cache_dtype: Optional[torch.dtype] = None,
        amp_dtype: Optional[torch.dtype] = None,
        impl: Optional[str] = None,
        generator: Optional[torch.Generator] = None,
        cache_manager: bool = False,
        decode_views: Optional[bool] = None,
    ) -> torch.Tensor:
        """Prompt prefill into a packed cache, then one cached forward per new
        token (bdh.py:1074-1193).  Returns (B, prompt + max_new_tokens) tokens.

        ``cache_manager=True`` uses ``CacheManager`` as bdh.py's generate builds
        it (compute fp32, storage ``cache_dtype``; bdh.py:1115-1123);
        ``decode_views`` is passed to it, and defaults to whether the decode
        runs on the HIP kernels."""
        B, P = idx.shape
        if cache_manager:
            if decode_views is None:
                decode_views = kernels.resolve_attn_impl(impl) == "hip"
            cache = CacheManager.from_config(self.config, batch_size=B, max_seq=P + max_new_tokens, device=idx.device,
                                             compute_dtype=torch.float32, storage_dtype=cache_dtype,
                                             decode_views=decode_views)
        else:
            dtype = cache_dtype or amp_dtype or torch.float32
            cache = KVCache(self.config, B, P + max_new_tokens, dtype, idx.device)
        out = torch.empty(B, P + max_new_tokens, dtype=idx.dtype, device=idx.device)
        out[:, :P] = idx
        ctx = (torch.autocast(idx.device.type, dtype=amp_dtype) if amp_dtype is not None
               else torch.autocast(idx.device.type, enabled=False))
        with ctx:
            logits, _ = self(idx, cache=cache, impl=impl, last_only=True)
            for t in range(max_new_tokens):
                nxt = self.sample(logits[:, -1].float(), temperature, top_k, generator)
                out[:, P + t] = nxt[:, 0]
                logits, _ = self(nxt, cache=cache, impl=impl, last_only=True)
        return out


__all__ = ["BDHConfig", "BDH", "KVCache"]
