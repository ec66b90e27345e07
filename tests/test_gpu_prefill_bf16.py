"""GPU parity of the bf16 prefill path (256x256 split-K score tiles, LDS-DMA
stream, RoPE from cos/sin made in the kernel (relative) or a per-call table
(absolute)) against the CPU oracle.

These shapes all qualify for that path (bf16, N a multiple of 64, 16-byte
aligned rows): ragged and exact multiples of the 256-row tile, one to five
row tiles, slab counts that are and are not multiples of 8 (the XCD grouping),
split-K from 1 to 8, q != k, permuted views, fused RoPE with a start offset and
the RoPE(x) copy.  Tolerance: bf16 2e-2 relative Frobenius; row 0 exactly 0.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, latent, normal, np_of, rel_fro, to_dev

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402

DEV = "cuda"
BF = torch.bfloat16


def _bf(a):
    return O.bf16_round(a)


SHAPES = [
    # B, H, T, N, D, Hv
    (1, 1, 1, 64, 16, 1),  # one row, one split
    (1, 1, 256, 128, 64, 1),  # exactly one tile, split 2 (N=128)
    (1, 1, 300, 512, 64, 1),  # ragged second tile, high split factor
    (3, 1, 257, 256, 32, 1),  # slab count 3 (not a multiple of 8)
    (2, 4, 512, 1024, 256, 1),  # C1-like layout, split 8
    (1, 2, 1100, 192, 40, 2),  # five row tiles, per-head V
]


@pytest.mark.parametrize("shape", SHAPES)
def test_bf16_self_attention_matches_oracle(shape):
    B, H, T, N, D, Hv = shape
    q = _bf(latent((B, H, T, N), 0))
    v = _bf(normal((B, Hv, T, D), 1))
    got = np_of(ext.tril_score_v(to_dev(q, BF), to_dev(q, BF), to_dev(v, BF)))
    want = O.tril_score_v_cpu(q, q, v)
    print(f"self {shape}: rel {rel_fro(got, want):.3e}", flush=True)
    assert rel_fro(got, want) <= TOL[BF]
    assert not got[:, :, 0].any()


@pytest.mark.parametrize("shape", SHAPES[1:4])
def test_bf16_distinct_q_k_matches_oracle(shape):
    B, H, T, N, D, Hv = shape
    q = _bf(latent((B, H, T, N), 0))
    k = _bf(latent((B, H, T, N), 5))
    v = _bf(normal((B, Hv, T, D), 1))
    got = np_of(ext.tril_score_v(to_dev(q, BF), to_dev(k, BF), to_dev(v, BF)))
    want = O.tril_score_v_cpu(q, k, v)
    assert rel_fro(got, want) <= TOL[BF]
    assert not got[:, :, 0].any()


def test_bf16_permuted_latent_view_and_fp32_v():
    """x_sparse as bdh.py makes it: a (B,T,nh,N) buffer viewed as (B,nh,T,N)."""
    B, T, H, N, D = 2, 333, 3, 128, 48
    x_bthn = _bf(latent((B, T, H, N), 3))
    xt = to_dev(x_bthn, BF).permute(0, 2, 1, 3)
    v = normal((B, 1, T, D), 4)
    got = np_of(ext.tril_score_v(xt, xt, to_dev(v, torch.float32)))
    xq = np.ascontiguousarray(x_bthn.transpose(0, 2, 1, 3))
    want = O.tril_score_v_cpu(xq, xq, _bf(v))
    assert rel_fro(got, want) <= TOL[BF]


@pytest.mark.parametrize("shape,start", [((1, 2, 300, 256, 64), 0), ((2, 1, 520, 512, 32), 17), ((1, 1, 1, 64, 8), 3)])
def test_bf16_fused_rope_matches_oracle(shape, start):
    B, H, T, N, D = shape
    x = _bf(latent((B, H, T, N), 0))
    v = _bf(normal((B, 1, T, D), 1))
    freqs = O.get_freqs(N)
    want, qr_want = O.tril_rope_score_v(x, v, freqs, start, bf16=True)
    qr = torch.full((B, H, T, N), float("nan"), dtype=BF, device=DEV)
    got = np_of(ext.tril_rope_score_v(to_dev(x, BF), to_dev(v, BF), torch.from_numpy(freqs).to(DEV), start,
                                      qr_out=qr))
    print(f"rope {shape} start {start}: rel {rel_fro(got, want):.3e} qr {rel_fro(np_of(qr), qr_want):.3e}",
          flush=True)
    assert rel_fro(got, want) <= TOL[BF]
    assert not got[:, :, 0].any()
    assert np.isfinite(np_of(qr)).all()  # every element of RoPE(x) was written
    assert rel_fro(np_of(qr), qr_want) <= 8e-3


@pytest.mark.parametrize("shape,start", [((1, 2, 300, 256, 64), 0), ((2, 1, 520, 512, 32), 17), ((1, 1, 1, 64, 8), 3),
                                         ((1, 1, 700, 256, 16), 5), ((1, 1, 1100, 128, 8), 2)])
def test_bf16_fused_rope_relative_table_matches_oracle(shape, start):
    """Without the RoPE(x) copy the kernel rotates each tile's rows about the
    tile's centre (scores depend only on position differences): single and
    paired diagonal tiles, full tiles at distances 1 to 4, rope_start > 0."""
    B, H, T, N, D = shape
    x = _bf(latent((B, H, T, N), 5))
    v = _bf(normal((B, 1, T, D), 6))
    freqs = O.get_freqs(N)
    want, _ = O.tril_rope_score_v(x, v, freqs, start, bf16=True)
    got = np_of(ext.tril_rope_score_v(to_dev(x, BF), to_dev(v, BF), torch.from_numpy(freqs).to(DEV), start))
    print(f"rope relative {shape} start {start}: rel {rel_fro(got, want):.3e}", flush=True)
    assert rel_fro(got, want) <= TOL[BF]
    assert not got[:, :, 0].any()


def test_bf16_fused_rope_full_c1_properties():
    """C1 at full size (B=8 nh=4 T=512 N=8192 D=256): size-independent checks.

    Exact homogeneity (both scalings are exact in bf16 and fp32, so the bits
    must match): out(x, 2v) = 2 out(x, v) and out(2x, v) = 4 out(x, v); row 0
    exactly zero; and batch element 0 against the oracle.
    """
    B, H, T, N, D = 8, 4, 512, 8192, 256
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.relu(0.32 * torch.randn(B, H, T, N, generator=g, device=DEV)).to(BF)
    v = torch.randn(B, 1, T, D, generator=g, device=DEV).to(BF)
    f = torch.from_numpy(O.get_freqs(N)).to(DEV)

    def run(xx, vv):
        o = torch.empty(B, H, T, D, dtype=torch.float32, device=DEV)
        return ext.tril_rope_score_v(xx, vv, f, 0, out=o)

    o1 = run(x, v)
    assert torch.equal(run(x, v * 2), o1 * 2)
    assert torch.equal(run(x * 2, v), o1 * 4)
    assert not o1[:, :, 0].any().item()
    want, _ = O.tril_rope_score_v(np_of(x[:1]), np_of(v[:1]), O.get_freqs(N), 0, bf16=True)
    assert rel_fro(np_of(o1[:1]), want) <= TOL[BF]


def _ran_score_tiles(fn):
    ext.profile_enable(True)
    try:
        out = fn()
        names = {n for n, _ in ext.profile_collect()}
    finally:
        ext.profile_enable(False)
    # the score-tile kernel, alone or with score x V fused into its tail
    assert names & {"k_sy_scores", "k_sy_scores_paired", "k_sy_scores_sv"}, names
    return out


@pytest.mark.parametrize("mode", ["self", "distinct", "rope"])
def test_bf16_long_sequences_stay_on_score_tile_path(mode):
    """Sequences with more than 256 work items per slab (23-24 row tiles):
    the kernel derives each item from its workgroup index, so the 256x256
    tile path covers them; results against the oracle."""
    T = 5800 if mode == "distinct" else 6000
    B, H, N, D = 1, 1, 64, 16
    print(f"long {mode} T={T}", flush=True)
    x = _bf(latent((B, H, T, N), 8))
    v = _bf(normal((B, 1, T, D), 9))
    if mode == "self":
        got = _ran_score_tiles(lambda: ext.tril_score_v(to_dev(x, BF), to_dev(x, BF), to_dev(v, BF)))
        want = O.tril_score_v_cpu(x, x, v)
    elif mode == "distinct":
        k = _bf(latent((B, H, T, N), 10))
        got = _ran_score_tiles(lambda: ext.tril_score_v(to_dev(x, BF), to_dev(k, BF), to_dev(v, BF)))
        want = O.tril_score_v_cpu(x, k, v)
    else:
        freqs = O.get_freqs(N)
        f = torch.from_numpy(freqs).to(DEV)
        got = _ran_score_tiles(lambda: ext.tril_rope_score_v(to_dev(x, BF), to_dev(v, BF), f, 3))
        want, _ = O.tril_rope_score_v(x, v, freqs, 3, bf16=True)
    g = np_of(got)
    assert rel_fro(g, want) <= TOL[BF]
    assert not g[:, :, 0].any()


@pytest.mark.parametrize("mode", ["self", "rope", "past"])
@pytest.mark.parametrize("D", [392, 512])
def test_bf16_wide_v_runs_score_tiles_per_256_columns(mode, D):
    """V wider than 256 columns (C5: D = 512): the score tiles are computed
    once and score x V runs once per 256 columns (the last slice ragged at
    D = 392); results against the oracle, fp32 V for the fused-RoPE case."""
    B, H, T, N = 2, 2, 300, 256
    print(f"wide V {mode} D={D}", flush=True)
    x = _bf(latent((B, H, T, N), 23))
    v = _bf(normal((B, 1, T, D), 24))
    if mode == "self":
        fn = lambda: ext.tril_score_v(to_dev(x, BF), to_dev(x, BF), to_dev(v, BF))  # noqa: E731
        want = O.tril_score_v_cpu(x, x, v)
    elif mode == "rope":
        freqs = O.get_freqs(N)
        f = torch.from_numpy(freqs).to(DEV)
        fn = lambda: ext.tril_rope_score_v(to_dev(x, BF), to_dev(v, torch.float32), f, 0)  # noqa: E731
        want, _ = O.tril_rope_score_v(x, v, freqs, 0, bf16=True)
    else:
        past = 100
        xd = to_dev(x, BF)
        fn = lambda: ext.tril_score_v_past(xd[:, :, past:], xd, to_dev(v, BF), past)  # noqa: E731
        want = O.tril_score_v_past(x[:, :, past:], x, v, past)
    got = np_of(_ran_score_tiles(fn))
    assert rel_fro(got, want) <= TOL[BF]



@pytest.mark.parametrize("N,table", [(16384, False), (16448, True)])
def test_bf16_fused_rope_stage_limit(N, table):
    """Without the RoPE(x) copy the score kernel makes cos/sin from 16
    frequencies per stage kept in 32 KB of LDS, so at most 512 stages per
    workgroup: 256 slabs of T = 2 run one split, so N = 16384 (512 stages)
    fills it and N = 16448 (514) takes the absolute-position table instead.
    Both against the oracle; the kernel profile shows which path ran."""
    B, H, T, D = 8, 32, 2, 16
    print(f"stage limit N={N}", flush=True)
    x = _bf(latent((B, H, T, N), 41))
    v = _bf(normal((B, 1, T, D), 42))
    freqs = O.get_freqs(N)
    want, _ = O.tril_rope_score_v(x, v, freqs, 5, bf16=True)
    ext.profile_enable(True)
    try:
        got = np_of(ext.tril_rope_score_v(to_dev(x, BF), to_dev(v, BF), torch.from_numpy(freqs).to(DEV), 5))
        names = {n for n, _ in ext.profile_collect()}
    finally:
        ext.profile_enable(False)
    assert names & {"k_sy_scores", "k_sy_scores_paired", "k_sy_scores_sv"} and ("k_rope_table" in names) == table, names
    assert rel_fro(got, want) <= TOL[BF]
    assert not got[:, :, 0].any()



REPRO_SHAPES = [
    # B, H, T, N, D, Hv, v dtype, out dtype
    (1, 1, 300, 512, 64, 1, BF, BF),  # two row tiles, split 8
    (2, 4, 512, 1024, 256, 1, BF, BF),  # C1 layout
    (1, 2, 700, 256, 96, 2, BF, torch.float32),  # three row tiles, a lone diagonal tile
    (3, 1, 257, 256, 32, 1, torch.float32, BF),  # fp32 V, one-row second tile
]


@pytest.mark.parametrize("shape", REPRO_SHAPES)
def test_score_v_matches_oracle_and_is_reproducible(shape):
    """Split-K self attention, with and without fused RoPE: against the oracle,
    and repeated calls give the same bits (the split sums run in a fixed order)."""
    B, H, T, N, D, Hv, vdt, odt = shape
    print(f"score x V reproducible {shape}", flush=True)
    x = _bf(latent((B, H, T, N), 51))
    v = normal((B, Hv, T, D), 52)
    v = _bf(v) if vdt == BF else v
    xd, vd = to_dev(x, BF), to_dev(v, vdt)
    freqs = O.get_freqs(N)
    fd = torch.from_numpy(freqs).to(DEV)

    def call(rope):
        if rope:
            return ext.tril_rope_score_v(xd, vd, fd, 3, out=torch.empty(B, H, T, D, dtype=odt, device=DEV))
        return ext.tril_score_v(xd, xd, vd)

    for rope in (False, True):
        first = call(rope)
        for _ in range(3):
            assert torch.equal(call(rope), first)
        want = O.tril_rope_score_v(x, v, freqs, 3, bf16=True)[0] if rope else O.tril_score_v_cpu(x, x, v)
        err = rel_fro(np_of(first), want)
        print(f"  rope={rope}: rel {err:.3e}", flush=True)
        assert err <= TOL[BF]
        assert not first[:, :, 0].any().item()


@pytest.mark.parametrize("B,H,T,N", [(2, 4, 512, 8192), (1, 2, 300, 16384), (3, 2, 700, 16384)])
def test_bf16_fused_rope_paired_stages_on_64k_rows(B, H, T, N):
    """Token rows a multiple of 64 KB apart (the model's (B, T, nh, N) x_sparse with nh*N a
    multiple of 32768) take the paired-stage score pass (both 64-byte halves of each 128-byte
    line requested together).  It loads the same rows and k chunks in another order, so the
    output, and the gradients the backward takes from the kept score tiles, equal those of the
    same x stored contiguously (the unpaired pass) bit for bit; ragged T included."""
    print(f"paired stages B={B} H={H} T={T} N={N}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(T + N)
    xt = torch.relu(0.3 * torch.randn(B, T, H, N, generator=g, device=DEV)).to(BF)
    assert (H * N * 2) % 65536 == 0
    x_perm = xt.permute(0, 2, 1, 3)
    x_cont = x_perm.contiguous()
    assert (N * 2) % 65536 != 0  # the contiguous copy takes the unpaired pass
    v = torch.randn(B, 1, T, 256, generator=g, device=DEV).to(BF)
    freqs = torch.from_numpy(O.get_freqs(N)).to(DEV)
    out_p, ws_p = ext.tril_rope_score_v_save(x_perm, v, freqs, 0)
    out_c, ws_c = ext.tril_rope_score_v_save(x_cont, v, freqs, 0)
    assert ws_p is not None and ws_c is not None
    assert torch.equal(out_p, out_c)
    d = torch.randn(B, H, T, 256, generator=g, device=DEV).to(BF)
    dx_p, dv_p = ext.tril_rope_score_v_bwd_saved(x_perm, v, d, freqs, 0, ws_p)
    dx_c, dv_c = ext.tril_rope_score_v_bwd_saved(x_cont, v, d, freqs, 0, ws_c)
    assert torch.equal(dv_p, dv_c)
    assert torch.equal(dx_p, dx_c)


# (B, H, T, N, D, permuted (B, T, H, N) rows)
SCHEDULE_SHAPES = [
    (8, 4, 512, 8192, 256, False),   # C1: 4 splits, full tile + diagonal pair
    (2, 3, 700, 1024, 64, False),    # three row tiles: a lone diagonal tile
    (1, 2, 300, 512, 128, False),    # ragged rows, 8 splits
    (3, 1, 1, 256, 64, False),       # one row
    (2, 2, 256, 2048, 256, False),   # one row tile (diagonal alone)
    (2, 4, 517, 8192, 256, True),    # 64 KB rows: paired stages
    (1, 8, 2048, 8192, 256, True),   # C5-like slab: one split, 256 stages, paired
]


@pytest.mark.parametrize("shape", SCHEDULE_SHAPES)
def test_bf16_fused_rope_schedules_agree(shape, monkeypatch):
    """The relative-RoPE score kernel's schedules (lockstep; ping-pong, two wave
    groups a barrier apart) run the same instructions in other orders: same DMA
    chunks, entries, rotations and MFMA sequence per accumulator.  Outputs and
    kept score tiles equal bit for bit; against the oracle within 2e-2."""
    B, H, T, N, D, perm = shape
    print(f"ping-pong vs lockstep {shape}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(T + N + D)
    if perm:
        x = torch.relu(0.32 * torch.randn(B, T, H, N, generator=g, device=DEV)).to(BF).permute(0, 2, 1, 3)
    else:
        x = torch.relu(0.32 * torch.randn(B, H, T, N, generator=g, device=DEV)).to(BF)
    v = torch.randn(B, 1, T, D, generator=g, device=DEV).to(BF)
    freqs = torch.from_numpy(O.get_freqs(N)).to(DEV)
    runs = {}
    for sched in ("lockstep", "pingpong"):
        monkeypatch.setenv("BDH_SY_SCHEDULE", sched)
        out, ws = ext.tril_rope_score_v_save(x, v, freqs, 3)
        assert ws is not None
        runs[sched] = (out, ws)
    assert torch.equal(runs["pingpong"][0], runs["lockstep"][0])
    # the kept tiles, through the saved backward's dV (the workspace's table
    # region is not written in the relative mode)
    d = torch.randn(B, H, T, D, generator=g, device=DEV).to(BF)
    dv = [ext.tril_rope_score_v_bwd_saved(x, v, d, freqs, 3, runs[k][1])[1] for k in ("lockstep", "pingpong")]
    assert torch.equal(dv[0], dv[1])
    b0 = np_of(x[:1])
    want, _ = O.tril_rope_score_v(b0, np_of(v[:1]), O.get_freqs(N), 3, bf16=True)
    assert rel_fro(np_of(runs["pingpong"][0][:1]), want) <= TOL[BF]
    assert not runs["pingpong"][0][:, :, 0].any().item()


@pytest.mark.parametrize("shape", [(8, 4, 512, 8192, 256), (2, 3, 700, 1024, 64), (1, 2, 300, 512, 128),
                                   (3, 1, 1, 256, 64), (16, 4, 1024, 8192, 256)])
def test_bf16_score_kernel_schedules_agree_without_rope(shape, monkeypatch):
    """The score kernel without RoPE (self attention on a pre-rotated QR and
    q != k) under the ping-pong and lockstep schedules: same bits; against the
    oracle within 2e-2 on batch element 0."""
    B, H, T, N, D = shape
    print(f"no-RoPE schedules {shape}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(T + N)
    x = torch.relu(0.32 * torch.randn(B, H, T, N, generator=g, device=DEV)).to(BF)
    k = torch.relu(0.32 * torch.randn(B, H, T, N, generator=g, device=DEV)).to(BF)
    v = torch.randn(B, 1, T, D, generator=g, device=DEV).to(BF)
    outs = {}
    for sched in ("lockstep", "pingpong"):
        monkeypatch.setenv("BDH_SY_SCHEDULE", sched)
        outs[sched] = (ext.tril_score_v(x, x, v), ext.tril_score_v(x, k, v))
    assert torch.equal(outs["pingpong"][0], outs["lockstep"][0])
    assert torch.equal(outs["pingpong"][1], outs["lockstep"][1])
    want = O.tril_score_v_eager(np_of(x[:1]), np_of(x[:1]), np_of(v[:1]))
    assert rel_fro(np_of(outs["pingpong"][0][:1]), want) <= TOL[BF]
    want = O.tril_score_v_eager(np_of(x[:1]), np_of(k[:1]), np_of(v[:1]))
    assert rel_fro(np_of(outs["pingpong"][1][:1]), want) <= TOL[BF]
