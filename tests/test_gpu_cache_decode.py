"""GPU parity of the decode step as the reference's cache delivers it.

* ``k_decode_f32q`` (fp32 arithmetic; fp32 or bf16 keys; q of either dtype)
  over every q / key / V dtype pair on capacity-strided views, against the
  oracle on the exact stored values: within 1e-5 when the output is fp32
  (the inputs are exact, only fp32 summation order differs), 2e-2 when it is
  rounded to bf16.
* The literal reference route at C3 size (B=64 nh=4 N=8192 D=256, S=511,
  bf16 storage, fp32 compute): bf16 q rotated into the slot, the past as
  ``CacheManager.get_past`` casts it up to fp32 (bdh_cache.py:238-243), into
  ``bdh_attn_decode(impl="hip")``; and the same step on the storage-dtype
  views this package's ``CacheManager`` hands the HIP decode.  Batch element
  0 against the oracle; both routes agree.
* The harness driven through ``CacheManager`` in bdh.py's call order
  (prefill, decode steps, a chunk after a past), fp32 and bf16 storage,
  with and without autocast, against its uncached forward.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, as_dtype_values, latent, normal, np_of, rel_fro, to_dev
from oracle import bdh_model_oracle as M

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402  (fails loudly when the library is missing)
import bdh_harness as H  # noqa: E402
import kernels  # noqa: E402
from bdh_cache import CacheManager  # noqa: E402

DEV = "cuda"
F32, BF = torch.float32, torch.bfloat16


def _decode_names(fn):
    ext.profile_enable(True)
    try:
        out = fn()
        names = {n for n, _ in ext.profile_collect()}
    finally:
        ext.profile_enable(False)
    return out, names


@pytest.mark.parametrize("qdt,kdt,vdt", [(F32, F32, F32), (BF, F32, F32), (F32, BF, BF), (F32, BF, F32),
                                         (BF, F32, BF), (F32, F32, BF)])
@pytest.mark.parametrize("S,N,D", [(1, 256, 32), (63, 768, 64), (64, 1536, 256), (65, 1024, 96),
                                   (200, 8192, 256)])
def test_f32_decode_all_dtype_pairs(qdt, kdt, vdt, S, N, D):
    print(f"f32q decode q={qdt} k={kdt} v={vdt} S={S} N={N} D={D}", flush=True)
    if N % (512 if kdt == BF else 256):
        pytest.skip("N outside the streaming kernel's widths")
    B, H, cap = 2, 3, S + 9
    kbuf = as_dtype_values(latent((B, H, cap, N), 2), kdt)
    vbuf = as_dtype_values(normal((B, 1, cap, D), 3), vdt)
    q = as_dtype_values(latent((B, H, 1, N), 4), qdt)
    kt, vt = to_dev(kbuf, kdt), to_dev(vbuf, vdt)
    got, names = _decode_names(lambda: ext.tril_decode(to_dev(q, qdt), kt.narrow(2, 0, S), vt.narrow(2, 0, S)))
    assert "k_decode_f32q" in names, names
    assert got.dtype == qdt
    want = O.tril_decode_cpu(q, kbuf[:, :, :S], vbuf[:, :, :S])
    err = rel_fro(np_of(got), want)
    print(f"  rel {err:.2e}", flush=True)
    assert err <= (1e-5 if qdt == F32 else TOL[BF])


@pytest.fixture(scope="module")
def c3_cache():
    """bf16 storage at C3 size; row S is the new token's RoPE(x) slot."""
    B, H, N, D, S, cap = 64, 4, 8192, 256, 511, 512
    g = torch.Generator(device=DEV).manual_seed(21)
    cm = CacheManager(1, cap, B, H, N, D, DEV, compute_dtype=F32, storage_dtype=BF, decode_views=False)
    kr, v = cm.reserve(0, S)
    kr.copy_(torch.relu(0.32 * torch.randn(B, H, S, N, generator=g, device=DEV)))
    v.copy_(torch.randn(B, 1, S, D, generator=g, device=DEV))
    cm.commit()
    x = torch.relu(0.32 * torch.randn(B, H, 1, N, generator=g, device=DEV)).to(BF)
    yield cm, x
    del cm
    torch.cuda.empty_cache()


def test_reference_cache_route_at_c3(c3_cache):
    """bdh.py:396-437 at a decode step with the reference's cache semantics:
    q = the bf16 RoPE'd token (paired rotation, bdh.py:396-405), past = fp32
    casts (bdh_cache.py:238-243)."""
    print("reference cache route at C3", flush=True)
    cm, x = c3_cache
    S, N = cm.seq_len, cm.n_latent
    f = kernels.get_freqs(N).to(DEV)
    cos, sin = kernels.rope_cos_sin(S + 1, 0, f)
    cp = cos.reshape(*cos.shape[:-1], -1, 2).narrow(-3, S, 1)
    sp = sin.reshape(*sin.shape[:-1], -1, 2).narrow(-3, S, 1)
    qr = kernels.bdh_rope_rotate_paired(x, cp, sp, impl="hip")
    assert qr.dtype == BF
    past_kr, past_v = cm.get_past(0)
    assert past_kr.dtype == F32 and past_v.dtype == F32  # the cast copies
    got, names = _decode_names(lambda: kernels.bdh_attn_decode(qr, past_kr, past_v, impl="hip"))
    assert "k_decode_f32q" in names, names
    cm.decode_views = True
    vk, vv = cm.get_past(0)
    assert vk.dtype == BF and vk.untyped_storage().data_ptr() == cm._kr_buf.untyped_storage().data_ptr()
    got_v, names_v = _decode_names(lambda: kernels.bdh_attn_decode(qr, vk, vv, impl="hip"))
    cm.decode_views = False
    assert "k_decode_bf16" in names_v, names_v
    assert got.dtype == BF and got_v.dtype == BF
    want = O.tril_decode_cpu(np_of(qr[:1]), np_of(vk[:1]), np_of(vv[:1]))
    e1, e2 = rel_fro(np_of(got[:1]), want), rel_fro(np_of(got_v[:1]), want)
    e12 = rel_fro(np_of(got_v), np_of(got))
    print(f"  cast route {e1:.2e}  storage views {e2:.2e}  between {e12:.2e}", flush=True)
    assert max(e1, e2, e12) <= TOL[BF]


def test_fp32_cache_route_at_c3_batch_slice():
    """The reference generate's default (cache_dtype=None: fp32 storage and
    compute, fp32 q) at C3 width on 8 batch rows, S=511."""
    print("fp32 cache route", flush=True)
    B, H, N, D, S = 8, 4, 8192, 256, 511
    k = latent((B, H, S + 1, N), 7)
    v = normal((B, 1, S + 1, D), 8)
    q = latent((B, H, 1, N), 9)
    kt, vt = to_dev(k, F32), to_dev(v, F32)
    got, names = _decode_names(lambda: kernels.bdh_attn_decode(to_dev(q, F32), kt.narrow(2, 0, S),
                                                               vt.narrow(2, 0, S), impl="hip"))
    assert "k_decode_f32q" in names, names
    want = O.tril_decode_cpu(q[:2], k[:2, :, :S], v[:2, :, :S])
    err = rel_fro(np_of(got[:2]), want)
    print(f"  rel {err:.2e}", flush=True)
    assert err <= 1e-5


def _model(p, mult):
    nh, D, N = p["encoder"].shape
    cfg = H.BDHConfig(n_layer=int(p["n_layer"]), n_embd=D, n_head=nh, mlp_internal_dim_multiplier=mult,
                      vocab_size=p["lm_head"].shape[1])
    m = H.BDH(cfg)
    with torch.no_grad():
        for k in ("encoder", "encoder_v", "decoder", "lm_head"):
            getattr(m, k).copy_(torch.from_numpy(p[k]))
        m.embed.weight.copy_(torch.from_numpy(p["embed"]))
    return m.to(DEV)


@pytest.mark.parametrize("storage,amp", [(None, False), (BF, False), (BF, True), (None, True)])
@pytest.mark.parametrize("views", [True, False])
def test_harness_through_cache_manager(storage, amp, views):
    print(f"harness via CacheManager storage={storage} amp={amp} views={views}", flush=True)
    p = M.init_params(2, 128, 2, 1024, 256, seed=15)
    m = _model(p, mult=16)
    idx = torch.from_numpy(np.random.default_rng(16).integers(0, 256, (2, 340))).to(DEV)
    ctx = torch.autocast("cuda", dtype=BF, enabled=amp)
    with torch.no_grad(), ctx:
        full, _ = m(idx, impl="hip")
        cm = CacheManager.from_config(m.config, 2, 340, DEV, compute_dtype=F32, storage_dtype=storage,
                                      page_size=128, decode_views=views)
        pre, _ = m(idx[:, :300], cache=cm, impl="hip")
        steps = [m(idx[:, t:t + 1], cache=cm, impl="hip")[0] for t in range(300, 303)]
        chunk, _ = m(idx[:, 303:340], cache=cm, impl="hip")
    assert cm.seq_len == 340 and cm.n_grows >= 1
    got = torch.cat([pre, *steps, chunk], dim=1).float().cpu().numpy()
    tol = 1e-4 if storage is None and not amp else 2e-2
    err = rel_fro(got, full.float().cpu().numpy())
    print(f"  rel {err:.2e}", flush=True)
    assert err <= tol
