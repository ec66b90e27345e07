"""GPU checks of the model harness on the HIP path.

* forward logits against the numpy model oracle: fp32 <= 1e-4, bf16 autocast
  <= 2e-2 (relative Frobenius), at one C2-width layer pair (D = 256, nh = 4,
  N = 8192, T = 512);
* the cached paths on the HIP kernels (fused prefill writing RoPE(x) into the
  cache, one-token decode over capacity-strided bf16 cache views, a chunk
  after a past on the score-tile path) against the uncached forward;
* a training step (cross entropy, backward through the HIP attention
  backward): at fp32 equal to the step with eager attention; under AMP, the
  bf16 attention's effect on the gradients (against the same AMP step with
  fp32 attention) no larger than that of the reference's eager bf16
  attention measured the same way;
* the training step's loss and gradients against the float64 model oracle;
* the C3 decode route at its model configuration (L=6, D=256, nh=4, N=8192,
  B=64, bf16 cache) through both caches: teacher-forced step logits against
  the model oracle at S = 256..263 and 504..511, and ``generate``'s draws
  against the oracle-anchored logits they were drawn from;
* ``generate`` end to end;
* the row LayerNorm (LN(y), LN(x + LN(y))) against F.layer_norm.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import rel_fro
from oracle import bdh_model_oracle as M

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402,F401  (fails loudly when the library is missing)
import bdh_harness as H  # noqa: E402

DEV = "cuda"


def _model(p, mult, device=DEV):
    nh, D, N = p["encoder"].shape
    cfg = H.BDHConfig(n_layer=int(p["n_layer"]), n_embd=D, n_head=nh, mlp_internal_dim_multiplier=mult,
                      vocab_size=p["lm_head"].shape[1])
    m = H.BDH(cfg)
    with torch.no_grad():
        for k in ("encoder", "encoder_v", "decoder", "lm_head"):
            getattr(m, k).copy_(torch.from_numpy(p[k]))
        m.embed.weight.copy_(torch.from_numpy(p["embed"]))
    return m.to(device)


def test_forward_fp32_matches_oracle():
    print("harness fp32 forward", flush=True)
    p = M.init_params(2, 64, 2, 256, 256, seed=11)
    m = _model(p, mult=8)
    idx = np.random.default_rng(12).integers(0, 256, (2, 300))
    with torch.no_grad():
        got, _ = m(torch.from_numpy(idx).to(DEV), impl="hip")
    assert rel_fro(got.cpu().numpy(), M.bdh_forward(p, idx)) <= 1e-4


def test_forward_bf16_c2_width_matches_oracle():
    print("harness bf16 forward, C2 width", flush=True)
    p = M.init_params(2, 256, 4, 8192, 256, seed=13)
    m = _model(p, mult=128)
    idx = np.random.default_rng(14).integers(0, 256, (2, 512))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        got, _ = m(torch.from_numpy(idx).to(DEV), impl="hip")
    assert got.dtype == torch.bfloat16
    assert rel_fro(got.float().cpu().numpy(), M.bdh_forward(p, idx)) <= 2e-2


def test_forward_full_c2_config_matches_oracle():
    """The C2 model configuration in full (6 layers, D=256, nh=4, N=8192, T=512)
    on two sequences, bf16 autocast, against the numpy model oracle (fp32):
    logits within 2e-2."""
    print("harness C2 config forward", flush=True)
    p = M.init_params(6, 256, 4, 8192, 256, seed=31)
    m = _model(p, mult=128)
    idx = np.random.default_rng(32).integers(0, 256, (2, 512))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        got, _ = m(torch.from_numpy(idx).to(DEV), impl="hip")
    assert rel_fro(got.float().cpu().numpy(), M.bdh_forward(p, idx)) <= 2e-2


@pytest.mark.parametrize("pad", [0, None])
def test_forward_c2_batch_paired_plan_matches_oracle(pad, monkeypatch):
    """The C2 configuration at its own batch (B=32, T=512, 6 layers): 128 slabs
    of two items each fill the chip at one split.  With x_sparse token rows
    unpadded (64 KB apart) the score pass runs the paired-stage kernel at split
    1; with the harness's padded rows (the default) the plain one (checked in
    the launch log).  Sequences 0 and 31 against the numpy model oracle within
    2e-2, and the two forwards give the same logits."""
    print(f"harness C2 batch forward (pad {pad})", flush=True)
    if pad is not None:
        monkeypatch.setattr(H, "_XS_PAD", pad)
    p = M.init_params(6, 256, 4, 8192, 256, seed=33)
    m = _model(p, mult=128)
    idx = np.random.default_rng(34).integers(0, 256, (32, 512))
    ext.profile_enable(True)
    try:
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            got, _ = m(torch.from_numpy(idx).to(DEV), impl="hip")
        torch.cuda.synchronize()
        names = {n for n, _ in ext.profile_collect()}
    finally:
        ext.profile_enable(False)
    assert ("k_sy_scores_paired" if pad == 0 else "k_sy_scores") in names, names
    assert "k_relu_enc" in names and "k_gated_dec" in names, names
    assert rel_fro(got[[0, 31]].float().cpu().numpy(), M.bdh_forward(p, idx[[0, 31]])) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cached_paths_match_uncached_forward(dtype):
    print(f"harness cached paths {dtype}", flush=True)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    p = M.init_params(2, 128, 2, 1024, 256, seed=15)
    m = _model(p, mult=16)
    idx = torch.from_numpy(np.random.default_rng(16).integers(0, 256, (2, 340))).to(DEV)
    amp = torch.autocast("cuda", dtype=torch.bfloat16, enabled=dtype == torch.bfloat16)
    with torch.no_grad(), amp:
        full, _ = m(idx, impl="hip")
        cache = H.KVCache(m.config, 2, 340, dtype, DEV)
        pre, _ = m(idx[:, :300], cache=cache, impl="hip")    # fused prefill into the cache
        steps = [m(idx[:, t:t + 1], cache=cache, impl="hip")[0] for t in range(300, 303)]  # decode
        chunk, _ = m(idx[:, 303:340], cache=cache, impl="hip")  # chunk after a past
    got = torch.cat([pre, *steps, chunk], dim=1).float().cpu().numpy()
    assert rel_fro(got, full.float().cpu().numpy()) <= tol


def _grads(p, idx, tgt, impl, amp, device=DEV, fp32_attention=False):
    """Parameter gradients (and the loss) of one training step.  With
    ``fp32_attention`` the layer's RoPE + attention runs in fp32 whatever the
    autocast state (on the GPU through the HIP fp32 kernels, on the CPU through
    torch), while every other product keeps its autocast dtype."""
    m = _model(p, mult=8, device=device)
    idx, tgt = idx.to(device), tgt.to(device)
    orig_rope, orig_attn, orig_rot = H.kernels.bdh_attn_rope, H.kernels.bdh_attn, H.kernels.bdh_rope_rotate
    if fp32_attention:
        def rope32(x, v, freqs, rope_start=0, **kw):
            with torch.autocast(torch.device(device).type, enabled=False):
                return orig_rope(x.float(), v.float(), freqs, rope_start, impl=kw.get("impl"))

        def attn32(q, k, v, **kw):
            with torch.autocast(torch.device(device).type, enabled=False):
                qf = q.float()
                return orig_attn(qf, qf if k is q else k.float(), v.float(), impl=kw.get("impl"))

        def rot32(x, cos, sin, out=None, **kw):
            assert out is None
            with torch.autocast(torch.device(device).type, enabled=False):
                return orig_rot(x.float(), cos, sin, impl=kw.get("impl"))

        H.kernels.bdh_attn_rope, H.kernels.bdh_attn, H.kernels.bdh_rope_rotate = rope32, attn32, rot32
    try:
        with torch.autocast(torch.device(device).type, dtype=torch.bfloat16, enabled=amp):
            _, loss = m(idx, tgt, impl=impl)
        loss.backward()
    finally:
        H.kernels.bdh_attn_rope, H.kernels.bdh_attn, H.kernels.bdh_rope_rotate = orig_rope, orig_attn, orig_rot
    g = {n: q.grad.float().cpu().numpy() for n, q in m.named_parameters()}
    g["loss"] = np.array([loss.item()])
    return g


@pytest.mark.parametrize("amp", [False, True])
def test_train_step_gradients(amp):
    """fp32: HIP attention gradients equal eager attention's (1e-4).

    AMP: the attention's own precision is isolated by holding everything else
    fixed.  The HIP step (bf16 attention) is compared with the same AMP step
    whose attention runs in fp32 (same device, same bf16 GEMMs); its effect on
    every gradient must be no larger than the effect of the reference's own
    AMP attention (eager: RoPE products and S rounded to bf16) measured the
    same way, eager bf16 against eager fp32 attention, within a factor 1.5:
    the two are different bf16 roundings of the same products, and their
    effects on this two-layer model's gradients differ by chance (measured:
    decoder 3.5e-2 against 3.0e-2).  That effect is 3-5e-2 on the weight
    gradients at this shape: at the model level the reference's AMP attention
    already moves gradients by more than the op-level 2e-2, which the attention
    op itself meets (C4 and the backward tests).  The eager pair runs on the
    CPU: its autograd makes bf16 batched products on transposed views, which
    have faulted ROCm GPUs."""
    print(f"harness train step amp={amp}", flush=True)
    p = M.init_params(2, 64, 2, 256, 256, seed=17)
    idx = torch.from_numpy(np.random.default_rng(18).integers(0, 256, (2, 200))).to(DEV)
    tgt = torch.from_numpy(np.random.default_rng(19).integers(0, 256, (2, 200))).to(DEV)
    if not amp:
        ref = _grads(p, idx, tgt, "eager", False)
        hip = _grads(p, idx, tgt, "hip", False)
        for n in ref:
            assert rel_fro(hip[n], ref[n]) <= 1e-4, n
        return
    hip = _grads(p, idx, tgt, "hip", True)
    hip32 = _grads(p, idx, tgt, "hip", True, fp32_attention=True)
    eag = _grads(p, idx, tgt, "eager", True, device="cpu")
    eag32 = _grads(p, idx, tgt, "eager", True, device="cpu", fp32_attention=True)
    for n in hip:
        e_hip, e_eag = rel_fro(hip[n], hip32[n]), rel_fro(eag[n], eag32[n])
        print(f"  {n}: bf16 vs fp32 attention: hip {e_hip:.3e} eager {e_eag:.3e}", flush=True)
        assert e_hip <= max(2e-2, 1.5 * e_eag), n


@pytest.mark.parametrize("amp", [False, True])
def test_train_step_gradients_match_oracle(amp):
    """The training step's loss and parameter gradients (HIP attention forward
    and backward) against the float64 oracle's (``bdh_loss_grads``, autograd of
    bdh_baseline.py:109-151 with the mean cross entropy of train.py:997-1034).

    fp32: every gradient within 1e-4.  AMP: the bf16 products of the model
    itself (encoder, encoder_v, decoder, lm_head and their backward under
    autocast, as in the reference) move the gradients by 3-6e-2 from the
    float64 values whatever the attention does (measured on the CPU with
    reference-semantics eager attention, in bf16 and in fp32).  So each
    gradient's error against the oracle must stay within max(2e-2, 1.25x) the
    error of the reference-semantics AMP step (eager attention, on the CPU)
    against the same oracle, and the loss within 2e-2.

    The fp32 comparison is well posed only when no ReLU input sits within fp32
    rounding of zero: such an element takes either branch depending on the
    GEMM's summation order, and its one gradient then moves every gradient
    upstream by ~1e-3 (measured: one of 2e5 inputs flipped between the GPU and
    the CPU product on another token draw).  The tokens are drawn so the
    smallest ReLU input is 1.7e-5 of its tensor's RMS, ~30x the products'
    rounding, and the test checks that first."""
    print(f"harness train step vs oracle amp={amp}", flush=True)
    p = M.init_params(2, 64, 2, 256, 256, seed=17)
    idx_np = np.random.default_rng(47).integers(0, 256, (1, 128))
    tgt_np = np.random.default_rng(48).integers(0, 256, (1, 128))
    assert M.relu_margin(p, idx_np) >= 1e-5
    idx, tgt = torch.from_numpy(idx_np), torch.from_numpy(tgt_np)
    want_loss, want = M.bdh_loss_grads(p, idx_np, tgt_np)
    hip = _grads(p, idx, tgt, "hip", amp)
    names = {"embed.weight": "embed", "encoder": "encoder", "encoder_v": "encoder_v", "decoder": "decoder",
             "lm_head": "lm_head"}
    if not amp:
        assert abs(hip["loss"][0] - want_loss) <= 1e-5 * abs(want_loss)
        for n, k in names.items():
            e = rel_fro(hip[n], want[k])
            print(f"  {k}: fp32 step vs oracle {e:.3e}", flush=True)
            assert e <= 1e-4, k
        return
    eag = _grads(p, idx, tgt, "eager", True, device="cpu")
    assert abs(hip["loss"][0] - want_loss) <= 2e-2 * abs(want_loss)
    for n, k in names.items():
        e_hip, e_eag = rel_fro(hip[n], want[k]), rel_fro(eag[n], want[k])
        print(f"  {k}: AMP step vs oracle: hip {e_hip:.3e}, reference-semantics eager {e_eag:.3e}", flush=True)
        assert e_hip <= max(2e-2, 1.25 * e_eag), k


# The C3 model (L=6, D=256, nh=4, N=8192, byte vocab) and batch (B=64).
C3_BATCH = 64


def _c3_params():
    return M.init_params(6, 256, 4, 8192, 256, seed=41)


def _c3_cache(m, kind, cap):
    if kind == "kv":
        return H.KVCache(m.config, C3_BATCH, cap, torch.bfloat16, DEV)
    return H.CacheManager.from_config(m.config, batch_size=C3_BATCH, max_seq=cap, device=DEV,
                                      compute_dtype=torch.float32, storage_dtype=torch.bfloat16,
                                      decode_views=True)


def _teacher_forced(m, tokens, prompt, steps, cache):
    """generate's loop (bdh.py:1074-1193) with the next tokens given instead of
    sampled: the prompt prefill into the cache, then one cached step per token,
    under bf16 autocast.  Returns (B, steps + 1, V) fp32 logits: those after the
    prompt, then those after each forced token."""
    out = []
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        lg, _ = m(tokens[:, :prompt], cache=cache, impl="hip", last_only=True)
        out.append(lg[:, -1].float())
        for t in range(prompt, prompt + steps):
            lg, _ = m(tokens[:, t:t + 1], cache=cache, impl="hip", last_only=True)
            out.append(lg[:, -1].float())
    return torch.stack(out, 1)


_ORACLE_LOGITS: dict = {}


def _oracle_logits(p, tokens_np, key):
    if key not in _ORACLE_LOGITS:
        _ORACLE_LOGITS[key] = M.bdh_forward(p, tokens_np)
    return _ORACLE_LOGITS[key]


@pytest.mark.parametrize("kind", ["kv", "manager"])
@pytest.mark.parametrize("prompt", [256, 504])
def test_decode_teacher_forced_c3_matches_oracle(kind, prompt):
    """The C3 decode route at its model configuration and batch: a prompt
    prefill (fused kernel writing RoPE(x) into the bf16 cache), then 8 cached
    one-token steps over capacity-strided bf16 past views, through the
    harness's packed cache (``kv``) and through ``CacheManager`` as bdh.py's
    generate builds it (fp32 compute, bf16 storage handed out uncast).  Each
    step's logits for sequences 0 and 1 of 64 against one oracle forward over
    the same tokens, within 2e-2.  Prompt 256 covers S = 256..263 (C3's first
    steps); prompt 504 covers S = 504..511 (C3's last)."""
    steps = 8
    print(f"C3 teacher-forced decode, {kind} cache, prompt {prompt}", flush=True)
    p = _c3_params()
    m = _model(p, mult=128)
    tokens_np = np.random.default_rng(42).integers(0, 256, (C3_BATCH, prompt + steps))
    tokens = torch.from_numpy(tokens_np).to(DEV)
    cache = _c3_cache(m, kind, prompt + steps)
    got = _teacher_forced(m, tokens, prompt, steps, cache).cpu().numpy()
    want = _oracle_logits(p, tokens_np[:2], ("tf", prompt))[:, prompt - 1:]
    for j in range(steps + 1):
        e = rel_fro(got[:2, j], want[:, j])
        print(f"  position {prompt - 1 + j}: logits rel {e:.3e}", flush=True)
        assert e <= 2e-2, j
    del cache
    torch.cuda.empty_cache()


@pytest.mark.parametrize("kind", ["kv", "manager"])
def test_generate_c3_samples_from_oracle_anchored_logits(kind):
    """``generate`` at the C3 configuration (B=64, 256-token prompt, top_k=3,
    temperature 1, seeded sampler), 8 new tokens.  Replaying the generated
    stream through the same cached route gives the logits generate sampled
    from (the kernels are deterministic): every new token is among their top 3,
    and for sequences 0 and 1 they match one oracle forward over the generated
    stream within 2e-2."""
    prompt, steps = 256, 8
    print(f"C3 generate, {kind} cache", flush=True)
    p = _c3_params()
    m = _model(p, mult=128)
    idx = torch.from_numpy(np.random.default_rng(43).integers(0, 256, (C3_BATCH, prompt))).to(DEV)
    out = m.generate(idx, steps, temperature=1.0, top_k=3, amp_dtype=torch.bfloat16, cache_dtype=torch.bfloat16,
                     impl="hip", generator=torch.Generator(device=DEV).manual_seed(5),
                     cache_manager=kind == "manager")
    assert out.shape == (C3_BATCH, prompt + steps) and torch.equal(out[:, :prompt], idx)
    cache = _c3_cache(m, kind, prompt + steps)
    logits = _teacher_forced(m, out, prompt, steps - 1, cache)  # (B, steps, V): the logits of each draw
    top3 = torch.topk(logits, 3, dim=-1).indices
    drawn = out[:, prompt:]
    assert bool((top3 == drawn.unsqueeze(-1)).any(-1).all()), "a generated token is outside the top 3"
    want = M.bdh_forward(p, out[:2].cpu().numpy())[:, prompt - 1:prompt - 1 + steps]
    e = rel_fro(logits[:2].cpu().numpy(), want)
    print(f"  generated-stream logits vs oracle: rel {e:.3e}", flush=True)
    assert e <= 2e-2
    del cache
    torch.cuda.empty_cache()


def test_generate_end_to_end_bf16():
    print("harness generate", flush=True)
    p = M.init_params(2, 64, 2, 256, 256, seed=21)
    m = _model(p, mult=8)
    idx = torch.from_numpy(np.random.default_rng(22).integers(0, 256, (4, 64))).to(DEV)
    out = m.generate(idx, 16, top_k=3, amp_dtype=torch.bfloat16, impl="hip",
                     generator=torch.Generator(device=DEV).manual_seed(5))
    assert out.shape == (4, 80) and torch.equal(out[:, :64], idx)
    assert int(out.min()) >= 0 and int(out.max()) < 256


@pytest.mark.parametrize("dx,dy", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                   (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("N", [2048, 200, 37])
def test_relu_mul_equals_torch(dx, dy, N):
    """out = x * relu(y) with y the head-major (nh, B, T, N) tensor viewed as
    (B, T, nh, N): equal to torch's product in x's dtype (8-wide and ragged
    rows), NaN in y propagates like torch's relu."""
    print(f"relu_mul {dx} {dy} N={N}", flush=True)
    B, T, nh = 2, 33, 3
    g = torch.Generator(device=DEV).manual_seed(N)
    x = torch.randn(B, T, nh, N, generator=g, device=DEV).to(dx)
    y_hm = torch.randn(nh, B, T, N, generator=g, device=DEV).to(dy)
    y_hm[0, 0, 0, 0] = float("nan")
    y = y_hm.permute(1, 2, 0, 3)
    got = ext.relu_mul(x, y)
    want = (x.float() * torch.relu(y.float())).to(dx)
    assert got.shape == x.shape and got.dtype == dx and got.is_contiguous()
    assert torch.isnan(got[0, 0, 0, 0])
    assert torch.equal(got.nan_to_num(7.0), want.nan_to_num(7.0))
    with pytest.raises(RuntimeError):
        ext.relu_mul(x, x, out=x)  # out overlaps an input


@pytest.mark.parametrize("shape", [(2, 300, 2, 1000, 96), (1, 512, 4, 8192, 256), (3, 257, 3, 136, 64),
                                   (1, 1, 1, 8, 32)])
def test_gated_gemm_matches_reference(shape):
    """x * relu(y @ wt^T) per head against a CPU fp32 reference (the GEMM
    rounded to bf16 after the ReLU, as the kernel and the unfused GEMM do):
    ragged row and column tiles, C2 width, one token."""
    B, T, nh, N, K = shape
    print(f"gated_gemm {shape}", flush=True)
    g = torch.Generator().manual_seed(K + N)
    y = torch.randn(B, nh, T, K, generator=g).to(torch.bfloat16)
    wt = (0.1 * torch.randn(nh, N, K, generator=g)).to(torch.bfloat16)
    x = torch.relu(torch.randn(B, T, nh, N, generator=g)).to(torch.bfloat16)
    got = ext.gated_gemm(y.to(DEV), wt.to(DEV), x.to(DEV))
    lin = torch.matmul(y.float(), wt.float().transpose(1, 2).contiguous())  # (B, nh, T, N) on the CPU
    want = (x.float() * torch.relu(lin).to(torch.bfloat16).float().permute(0, 2, 1, 3)).to(torch.bfloat16)
    assert got.shape == x.shape and got.dtype == torch.bfloat16
    assert rel_fro(got.float().cpu().numpy(), want.float().numpy()) <= 1e-2


@pytest.mark.parametrize("shape,odt", [((64, 32768, 256), torch.bfloat16), ((3, 1000, 200), torch.float32),
                                       ((300, 640, 130), torch.bfloat16), ((1, 64, 8), torch.float32)])
def test_small_gemm_matches_reference(shape, odt):
    """Split-K few-row GEMM against a CPU fp32 product: the decode-step decoder
    shape, ragged K / D / row tiles, fp32 and bf16 outputs."""
    M, K, D = shape
    print(f"small_gemm {shape} {odt}", flush=True)
    g = torch.Generator().manual_seed(M + K)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    b = (0.05 * torch.randn(K, D, generator=g)).to(torch.bfloat16)
    got = ext.small_gemm(a.to(DEV), b.to(DEV), odt)
    want = a.float() @ b.float()
    assert got.shape == (M, D) and got.dtype == odt
    assert rel_fro(got.float().cpu().numpy(), want.numpy()) <= (1e-5 if odt == torch.float32 else 1e-2)


@pytest.mark.parametrize("D", [64, 256, 512, 1024])
@pytest.mark.parametrize("dy,dx,do", [(torch.bfloat16, None, torch.bfloat16), (torch.float32, None, torch.float32),
                                      (torch.bfloat16, torch.float32, torch.float32),
                                      (torch.float32, torch.bfloat16, torch.bfloat16)])
def test_layer_norm_rows_matches_reference(D, dy, dx, do):
    """LN(y) and LN(x + LN(y)) (no affine, eps 1e-5) against F.layer_norm in fp32
    on the CPU: fp32 outputs within 1e-5, bf16 outputs within bf16 rounding
    (2^-8 relative); y a permuted (strided) view; rows with a large offset."""
    print(f"layer_norm_rows D={D} y={dy} x={dx} out={do}", flush=True)
    g = torch.Generator().manual_seed(D)
    y = (3.0 * torch.randn(2, 37, 3, D, generator=g) + 100.0).to(dy)
    x = torch.randn(2, 3, 37, D, generator=g).to(dx) if dx is not None else None
    yv = y.to(DEV).permute(0, 2, 1, 3)  # (2, 3, 37, D), strided rows
    got = ext.layer_norm_rows(yv, x.to(DEV) if x is not None else None, out_dtype=do)
    ln = lambda t: F.layer_norm(t, (D,), eps=1e-5)  # noqa: E731
    want = ln(y.float().permute(0, 2, 1, 3))
    if x is not None:
        want = ln(x.float() + want)
    assert got.shape == want.shape and got.dtype == do
    tol = 1e-5 if do == torch.float32 else 2.0 ** -8
    assert rel_fro(got.float().cpu().numpy(), want.numpy()) <= tol


@pytest.mark.parametrize("D", [256, 512])
@pytest.mark.parametrize("dy", [torch.bfloat16, torch.float32])
def test_layer_norm_rows_bf16_second_output(D, dy):
    """``bdh_layer_norm_rows2``: the residual LN's fp32 output and its bf16 copy,
    the copy written into a strided view (a KV cache's V slot, rows capacity
    apart): the copy equals the fp32 output rounded to bf16 bit for bit, and the
    fp32 output equals the one-output entry point's.  Rows outside the view are
    untouched."""
    g = torch.Generator().manual_seed(D + 1)
    B, T, cap = 5, 3, 11
    y = torch.randn(B, T, D, generator=g).to(dy).to(DEV)
    x = torch.randn(B, T, D, generator=g).to(DEV)
    cache = torch.full((B, 1, cap, D), 7.0, dtype=torch.bfloat16, device=DEV)
    slot = cache[:, 0].narrow(1, 4, T)  # (B, T, D), rows cap * D apart
    out = ext.layer_norm_rows(y, x, out_dtype=torch.float32, out_bf16=slot)
    assert torch.equal(out, ext.layer_norm_rows(y, x, out_dtype=torch.float32))
    assert torch.equal(slot, out.to(torch.bfloat16))
    rest = torch.cat([cache[:, 0, :4], cache[:, 0, 4 + T:]], dim=1)
    assert bool((rest == 7.0).all())
    with pytest.raises(RuntimeError):
        ext.layer_norm_rows(y, x, out_dtype=torch.float32, out_bf16=torch.empty(B, T, D, device=DEV))  # fp32
