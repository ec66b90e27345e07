"""Packed KR/V decode cache with the reference's ``CacheManager`` interface
(bdh_cache.py:38-336), for ``bdh.py`` to import unchanged.

Layout, as the decode kernels read it in place:

* ``_kr_buf``: (n_layer, B, n_head, capacity, N) -- RoPE(x) rows;
* ``_v_buf``:  (n_layer, B, 1, capacity, D) -- V rows (one head, broadcast);

both in the storage dtype.  A forward over T tokens writes rows
``[seq_len, seq_len + T)`` of every layer (``reserve`` / ``append`` /
``stage``) and ``commit`` advances ``seq_len`` once all layers have written.
With ``page_size`` the buffers start at one page and grow geometrically
(at least doubling, page-aligned, capped at ``max_seq``) when a write needs
more rows; a grow invalidates earlier views.

The one difference from the reference: its ``get_past`` / ``stage`` cast a
narrower storage dtype up to ``compute_dtype`` on every call
(bdh_cache.py:238-243, 313-316) -- a full copy of the past per layer and
decode step.  When the decode runs on the HIP kernels they read the storage
dtype in place and widen it in registers (bf16 -> fp32 is exact, so the
products are those of the cast copy), and the copy is skipped.  ``decode_views``
picks the behaviour: ``None`` (default) hands storage-dtype views when
``BDH_ATTN_IMPL`` resolves to ``hip`` and the cache lives on a ROCm device,
``True`` always, ``False`` never (the reference's casts).  Under ``hip`` the
views are safe for every consumer bdh.py has: ``bdh_attn_decode`` takes mixed
q / past dtypes, and the multi-token continuation copies the past into a
buffer of QR's dtype (bdh.py:446-461).
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch


class CacheManager:
    """Layer-major packed KR/V cache (bdh_cache.py:38-111 interface)."""

    def __init__(
        self,
        n_layer: int,
        max_seq: int,
        batch_size: int,
        n_head: int,
        n_latent: int,
        n_embd: int,
        device: torch.device | str,
        *,
        compute_dtype: torch.dtype = torch.float32,
        storage_dtype: Optional[torch.dtype] = None,
        page_size: Optional[int] = None,
        decode_views: Optional[bool] = None,
    ):
        if max_seq < 1:
            raise ValueError("max_seq must be >= 1")
        if page_size is not None and page_size < 1:
            raise ValueError("page_size must be >= 1 when set")
        self.n_layer = int(n_layer)
        self.max_seq = int(max_seq)
        self.batch_size = int(batch_size)
        self.n_head = int(n_head)
        self.n_latent = int(n_latent)
        self.n_embd = int(n_embd)
        self.device = torch.device(device)
        self.compute_dtype = compute_dtype
        self.storage_dtype = storage_dtype or compute_dtype
        self.storage_matches_compute = self.storage_dtype == self.compute_dtype
        self.page_size = page_size
        self.decode_views = decode_views
        self.seq_len = 0
        self._pending_t: Optional[int] = None
        self.n_grows = 0
        self.bytes_copied_on_grow = 0
        self.capacity = self.max_seq if page_size is None else min(self.max_seq, int(page_size))
        self._kr_buf, self._v_buf = self._alloc(self.capacity, torch.zeros)

    @classmethod
    def from_config(
        cls,
        config,
        batch_size: int,
        max_seq: int,
        device: torch.device | str,
        *,
        compute_dtype: torch.dtype = torch.float32,
        storage_dtype: Optional[torch.dtype] = None,
        page_size: Optional[int] = None,
        decode_views: Optional[bool] = None,
    ) -> "CacheManager":
        """Sizes from a BDH config: N = mlp_internal_dim_multiplier * n_embd / n_head
        (bdh_cache.py:123-149)."""
        nh, D = int(config.n_head), int(config.n_embd)
        return cls(
            config.n_layer, max_seq, batch_size, nh, config.mlp_internal_dim_multiplier * D // nh, D, device,
            compute_dtype=compute_dtype, storage_dtype=storage_dtype, page_size=page_size,
            decode_views=decode_views,
        )

    # ------------------------------------------------------------ storage
    def _alloc(self, cap: int, fill):
        kr = fill(self.n_layer, self.batch_size, self.n_head, cap, self.n_latent,
                  dtype=self.storage_dtype, device=self.device)
        v = fill(self.n_layer, self.batch_size, 1, cap, self.n_embd, dtype=self.storage_dtype, device=self.device)
        return kr, v

    @property
    def _kr(self) -> List[torch.Tensor]:
        return list(self._kr_buf.unbind(0))

    @property
    def _v(self) -> List[torch.Tensor]:
        return list(self._v_buf.unbind(0))

    @property
    def bytes_allocated(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self._kr_buf, self._v_buf))

    @property
    def hands_storage_views(self) -> bool:
        """Whether ``get_past`` / ``stage`` return storage-dtype views (no cast copy).

        Only bf16 and fp32 storage is handed out uncast: those are the key and value
        dtypes the HIP decode reads.  Any other storage dtype (the reference documents
        float16, bdh.py:1096) keeps the reference's cast to the compute dtype."""
        if self.storage_matches_compute:
            return True
        if self.storage_dtype not in (torch.bfloat16, torch.float32):
            return False
        if self.decode_views is not None:
            return bool(self.decode_views)
        if self.device.type != "cuda" or torch.version.hip is None:
            return False
        from kernels.attention_dispatch import resolve_attn_impl

        return resolve_attn_impl() == "hip"

    def _next_capacity(self, need: int) -> int:
        ps = int(self.page_size)
        target = max(int(need), 2 * self.capacity)
        return min(self.max_seq, -(-target // ps) * ps)

    def _ensure_capacity(self, need: int) -> None:
        if need <= self.capacity:
            return
        if need > self.max_seq or self.page_size is None:
            raise RuntimeError(f"cache overflow: need {need} slots but max_seq={self.max_seq}")
        self._grow(self._next_capacity(need))

    def ensure_capacity(self, need: int) -> None:
        """Grow (when paging) so ``need`` rows fit; no-op when they already do."""
        self._ensure_capacity(need)

    def _grow(self, new_cap: int) -> None:
        if new_cap <= self.capacity:
            return
        kr, v = self._alloc(new_cap, torch.empty)  # rows past ``used`` are written before they are read
        used = self.seq_len + (self._pending_t or 0)
        if used:
            kr.narrow(3, 0, used).copy_(self._kr_buf.narrow(3, 0, used))
            v.narrow(3, 0, used).copy_(self._v_buf.narrow(3, 0, used))
            per_row = self.n_layer * self.batch_size * (self.n_head * self.n_latent + self.n_embd)
            self.bytes_copied_on_grow += used * per_row * self._kr_buf.element_size()
        self._kr_buf, self._v_buf = kr, v
        self.capacity = new_cap
        self.n_grows += 1

    # --------------------------------------------------------------- views
    def _rows(self, level: int, start: int, n: int) -> Tuple[torch.Tensor, torch.Tensor]:
        return self._kr_buf[level].narrow(2, start, n), self._v_buf[level].narrow(2, start, n)

    def _for_compute(self, kr: torch.Tensor, v: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        if self.hands_storage_views:
            return kr, v
        return kr.to(self.compute_dtype), v.to(self.compute_dtype)

    def get_past(self, level: int) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        """Rows ``[0, seq_len)`` of ``level`` as capacity-strided views, or
        ``(None, None)`` before the first commit (bdh_cache.py:226-244)."""
        if self.seq_len == 0:
            return None, None
        return self._for_compute(*self._rows(level, 0, self.seq_len))

    def _claim(self, T: int) -> int:
        """Make room for ``seq_len + T`` rows and record the pending width."""
        self._ensure_capacity(self.seq_len + T)
        if self._pending_t is None:
            self._pending_t = T
        elif self._pending_t != T:
            raise RuntimeError(f"inconsistent append T: layer wrote {T}, pending={self._pending_t}")
        return self.seq_len + T

    def reserve(self, level: int, T: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Writable storage-dtype views of rows ``[seq_len, seq_len + T)``
        (bdh_cache.py:258-277); may grow first."""
        if T < 1:
            raise ValueError("reserve T must be >= 1")
        self._claim(T)
        return self._rows(level, self.seq_len, T)

    def _write(self, level: int, new_kr: torch.Tensor, new_v: torch.Tensor) -> int:
        T = new_kr.size(2)
        if T != new_v.size(2):
            raise ValueError(f"kr T={T} != v T={new_v.size(2)}")
        end = self._claim(T)
        dst_kr, dst_v = self._rows(level, self.seq_len, T)
        dst_kr.copy_(new_kr)  # copy_ casts to the storage dtype
        dst_v.copy_(new_v)
        return end

    def append(self, level: int, new_kr: torch.Tensor, new_v: torch.Tensor) -> None:
        """Write this layer's new rows at ``seq_len`` (bdh_cache.py:294-296)."""
        self._write(level, new_kr, new_v)

    def stage(self, level: int, new_kr: torch.Tensor, new_v: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Write the new rows and return past + new as one view each
        (bdh_cache.py:298-317)."""
        end = self._write(level, new_kr, new_v)
        return self._for_compute(*self._rows(level, 0, end))

    def commit(self) -> None:
        """Advance ``seq_len`` by the width every layer wrote (bdh_cache.py:319-324)."""
        if self._pending_t is not None:
            self.seq_len += self._pending_t
            self._pending_t = None

    def reset(self) -> None:
        self.seq_len = 0
        self._pending_t = None
        self.n_grows = 0
        self.bytes_copied_on_grow = 0


__all__ = ["CacheManager"]
