"""CPU checks of ``bdh_cache.CacheManager`` (reference interface bdh_cache.py:38-336).

Known answers from the reference's own cache tests: capacity and footprint in
slot units (test_cache_pack.py:272-293), geometric paging 16 -> 512 in at most
six grows (:480-512), a single grow for ``ensure_capacity`` (:515-536), and
values kept across a grow between ``reserve`` and ``stage`` (:539-575).  Then
what this build changes: ``get_past`` / ``stage`` hand storage-dtype views
(no cast copy) only when the decode runs on the HIP kernels, and the harness
driven through ``CacheManager`` in bdh.py's call order produces the same
logits and tokens as its own cache.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import rel_fro
from oracle import bdh_model_oracle as M

import bdh_harness as H
from bdh_cache import CacheManager

CFG = H.BDHConfig(n_layer=2, n_embd=16, n_head=2, mlp_internal_dim_multiplier=4, vocab_size=9)
N = CFG.n_latent
STRIDE = CFG.n_layer * (CFG.n_head * N + CFG.n_embd) * 4  # fp32 bytes per slot over all layers


def _fill_tokenwise(cm, n, value=None):
    for _ in range(n):
        for level in range(CFG.n_layer):
            kr = torch.zeros(1, CFG.n_head, 1, N) if value is None else torch.full((1, CFG.n_head, 1, N), value)
            cm.append(level, kr, torch.zeros(1, 1, 1, CFG.n_embd))
        cm.commit()


def test_layout_and_footprint():
    cm = CacheManager.from_config(CFG, batch_size=3, max_seq=10, device="cpu")
    assert cm._kr_buf.shape == (2, 3, 2, 10, N) and cm._v_buf.shape == (2, 3, 1, 10, 16)
    assert cm.capacity == 10 and cm.seq_len == 0 and not cm._kr_buf.any()
    assert cm.get_past(0) == (None, None)
    assert cm._kr[1].data_ptr() == cm._kr_buf[1].data_ptr()
    cm = CacheManager.from_config(CFG, batch_size=1, max_seq=16, device="cpu", page_size=4)
    assert cm.capacity == 4 and cm.bytes_allocated == 4 * STRIDE
    _fill_tokenwise(cm, 16)
    assert cm.capacity == 16 and cm.bytes_allocated == 16 * STRIDE


def test_reserve_commit_and_views():
    cm = CacheManager.from_config(CFG, batch_size=1, max_seq=8, device="cpu")
    for level in range(CFG.n_layer):
        kr, v = cm.reserve(level, 3)
        kr.fill_(level + 1.0)
        v.fill_(-1.0)
    assert cm.seq_len == 0 and cm.get_past(0) == (None, None)
    cm.commit()
    assert cm.seq_len == 3
    kr, v = cm.get_past(1)
    assert kr.shape == (1, 2, 3, N) and bool((kr == 2.0).all()) and bool((v == -1.0).all())
    # capacity-strided views into the packed buffer, unit last stride
    assert kr.stride(2) == N and kr.stride(1) == 8 * N and kr.stride(-1) == 1
    assert kr.untyped_storage().data_ptr() == cm._kr_buf.untyped_storage().data_ptr()
    cm.reserve(0, 2)
    with pytest.raises(RuntimeError, match="inconsistent append T"):
        cm.reserve(1, 1)
    with pytest.raises(ValueError):
        cm.reserve(0, 0)
    with pytest.raises(RuntimeError, match="cache overflow"):
        cm.ensure_capacity(9)
    cm.reset()
    assert cm.seq_len == 0 and cm.get_past(0) == (None, None)


def test_geometric_paging_known_answers():
    cm = CacheManager.from_config(CFG, batch_size=1, max_seq=512, device="cpu", page_size=16)
    caps = []
    for _ in range(512):
        for level in range(CFG.n_layer):
            cm.append(level, torch.zeros(1, 2, 1, N), torch.zeros(1, 1, 1, 16))
        cm.commit()
        if not caps or caps[-1] != cm.capacity:
            caps.append(cm.capacity)
    assert caps == [16, 32, 64, 128, 256, 512] and cm.n_grows == 5
    # prefix recopied at each grow: 16 + 32 + 64 + 128 + 256 slots
    assert cm.bytes_copied_on_grow == (16 + 32 + 64 + 128 + 256) * STRIDE
    # partial final page: 37 slots in pages of 8 -> 8, 16, 32, 37
    cm = CacheManager.from_config(CFG, batch_size=1, max_seq=37, device="cpu", page_size=8)
    caps = [cm.capacity]
    for _ in range(37):
        _fill_tokenwise(cm, 1)
        if caps[-1] != cm.capacity:
            caps.append(cm.capacity)
    assert caps == [8, 16, 32, 37]
    with pytest.raises(RuntimeError, match="cache overflow"):
        _fill_tokenwise(cm, 1)


def test_ensure_capacity_single_grow():
    cm = CacheManager.from_config(CFG, batch_size=1, max_seq=256, device="cpu", page_size=8)
    cm.ensure_capacity(200)
    assert cm.n_grows == 1 and 200 <= cm.capacity <= 256
    _fill_tokenwise(cm, 200)
    assert cm.n_grows == 1 and cm.seq_len == 200


def test_values_survive_grow_between_reserve_and_stage():
    cm = CacheManager.from_config(CFG, batch_size=1, max_seq=64, device="cpu", page_size=4)
    for level in range(CFG.n_layer):
        cm.append(level, torch.full((1, 2, 4, N), 1.0), torch.full((1, 1, 4, 16), 2.0))
    cm.commit()
    for level in range(CFG.n_layer):
        kr, v = cm.reserve(level, 1)  # grows 4 -> 8 first
        kr.fill_(3.0)
        v.fill_(4.0)
    cm.commit()
    assert cm.n_grows == 1 and cm.capacity == 8
    kr, v = cm.get_past(0)
    assert bool((kr[:, :, :4] == 1).all()) and bool((kr[:, :, 4] == 3).all())
    assert bool((v[:, :, :4] == 2).all()) and bool((v[:, :, 4] == 4).all())
    for level in range(CFG.n_layer):
        kr, v = cm.stage(level, torch.full((1, 2, 5, N), 5.0), torch.full((1, 1, 5, 16), 6.0))  # 10 > 8: grows
    assert cm.capacity == 16 and kr.shape[2] == 10
    assert bool((kr[:, :, :4] == 1).all()) and bool((kr[:, :, 4] == 3).all()) and bool((kr[:, :, 5:] == 5).all())


def test_storage_views_policy(monkeypatch):
    """fp32 compute over bf16 storage: the reference casts the past up on every
    get_past (bdh_cache.py:238-243); here the cast is skipped when the decode
    runs on the HIP kernels, which read the bf16 rows in place."""
    import kernels.attention_dispatch as AD

    def past_dtype(cm):
        for level in range(CFG.n_layer):
            cm.append(level, torch.ones(1, 2, 2, N), torch.ones(1, 1, 2, 16))
        cm.commit()
        return cm.get_past(0)[0].dtype

    make = lambda **kw: CacheManager.from_config(  # noqa: E731
        CFG, 1, 8, "cpu", compute_dtype=torch.float32, storage_dtype=torch.bfloat16, **kw)
    assert past_dtype(make()) == torch.float32  # CPU cache: the reference's cast
    assert past_dtype(make(decode_views=False)) == torch.float32
    cm = make(decode_views=True)
    assert past_dtype(cm) == torch.bfloat16
    kr, _ = cm.get_past(1)
    assert kr.untyped_storage().data_ptr() == cm._kr_buf.untyped_storage().data_ptr()  # a view, no copy
    st, _ = cm.stage(0, torch.ones(1, 2, 1, N), torch.ones(1, 1, 1, 16))
    assert st.dtype == torch.bfloat16 and st.shape[2] == 3
    same = CacheManager.from_config(CFG, 1, 8, "cpu", storage_dtype=torch.float32)
    assert same.hands_storage_views and past_dtype(same) == torch.float32
    # default policy on a ROCm device follows BDH_ATTN_IMPL (explicit hip only)
    monkeypatch.setattr(torch.version, "hip", "7.0", raising=False)
    dev = make()
    dev.device = torch.device("cuda")
    for env, want in (("hip", True), ("eager", False)):
        monkeypatch.setenv("BDH_ATTN_IMPL", env)
        assert AD.resolve_attn_impl() == env
        assert dev.hands_storage_views is want
    # float16 storage (documented by the reference, bdh.py:1096): the HIP decode
    # reads only bf16/fp32 rows, so the past is cast to the compute dtype even
    # with the hip impl forced or views asked for.
    monkeypatch.setenv("BDH_ATTN_IMPL", "hip")
    for views in (None, True):
        half = CacheManager.from_config(CFG, 1, 8, "cpu", compute_dtype=torch.float32,
                                        storage_dtype=torch.float16, decode_views=views)
        half.device = torch.device("cuda")
        assert half.hands_storage_views is False
        half.device = torch.device("cpu")
        assert past_dtype(half) == torch.float32
        st, _ = half.stage(0, torch.ones(1, 2, 1, N), torch.ones(1, 1, 1, 16))
        assert st.dtype == torch.float32


def _model(seed=3):
    p = M.init_params(CFG.n_layer, CFG.n_embd, CFG.n_head, N, CFG.vocab_size, seed=seed)
    m = H.BDH(CFG)
    with torch.no_grad():
        for k in ("encoder", "encoder_v", "decoder", "lm_head"):
            getattr(m, k).copy_(torch.from_numpy(p[k]))
        m.embed.weight.copy_(torch.from_numpy(p["embed"]))
    return m


@pytest.mark.parametrize("storage", [None, torch.bfloat16])
def test_harness_through_cache_manager_matches_full_forward(storage):
    """bdh.py's call order (in-place RoPE into reserved slots when storage is
    the compute dtype; else get_past, attention, append) over prefill, a
    one-token step, a chunk after a past, and a paged grow."""
    m = _model()
    idx = torch.from_numpy(np.random.default_rng(6).integers(0, 9, (2, 14)))
    full, _ = m(idx, impl="eager")
    cm = CacheManager.from_config(CFG, 2, 14, "cpu", storage_dtype=storage, page_size=4)
    with torch.no_grad():
        pre, _ = m(idx[:, :6], cache=cm, impl="eager")
        step, _ = m(idx[:, 6:7], cache=cm, impl="eager")
        chunk, _ = m(idx[:, 7:11], cache=cm, impl="eager")
        last, _ = m(idx[:, 11:14], cache=cm, impl="eager", last_only=True)
    assert cm.seq_len == 14 and cm.n_grows >= 2
    got = torch.cat([pre, step, chunk], dim=1)
    tol = 1e-4 if storage is None else 3e-2
    assert rel_fro(got.numpy(), full[:, :11].detach().numpy()) <= tol
    assert rel_fro(last.numpy(), full[:, 13:14].detach().numpy()) <= tol


def test_generate_cache_manager_matches_own_cache():
    m = _model(seed=7)
    idx = torch.from_numpy(np.random.default_rng(8).integers(0, 9, (3, 5)))
    a = m.generate(idx, 6, top_k=3, impl="eager", generator=torch.Generator().manual_seed(1))
    b = m.generate(idx, 6, top_k=3, impl="eager", generator=torch.Generator().manual_seed(1), cache_manager=True)
    assert torch.equal(a, b)
