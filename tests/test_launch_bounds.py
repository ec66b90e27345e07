"""Host-side bounds of the library launches the model harness makes at the C2, C5 and C3 shapes.

CPU only: the launch plans and index formulas of the kernels the harness's
HIP legs run (csrc/syrk.hip: k_sy_scores work items, their x loads and
partial-tile stores, k_sy_sv's partial, V and output accesses;
csrc/decode.hip: k_decode_bf16's key, q and partial accesses; the training
backward's k_dq_sy B loads on x, k_dv_sy and k_dv_dma, the forward's k_sv_dma; csrc/model.hip: k_gated_gemm's
LDS-DMA operand loads and epilogue x loads; csrc/gated_dec.hip: k_gated_dec's
grid, operand DMA, LDS fragment reads and partial stores; csrc/enc.hip: k_relu_enc's grid,
encoder DMA, fragment and tile accesses and output stores) are restated here and evaluated over every
work item, with the strides of the views the harness passes (x_sparse as the
permuted (B, T, nh, N) encoder output, the packed KV cache's
capacity-strided past views).  Each access must fall inside its buffer and
every score tile must be computed exactly once.
"""

import numpy as np
import pytest

TILE, TILE_ELEMS = 256, 256 * 256
FULL, DIAG2, DIAG1 = 0, 1, 2

# (name, B, nh, T, N, D): the harness legs' attention shapes (bench.py C2, C5;
# C3's prompt prefill)
PREFILL = [("C2", 32, 4, 512, 8192, 256), ("C5", 4, 8, 2048, 8192, 512), ("C3 prompt", 64, 4, 256, 8192, 256)]


def sy_plan(nslab, T, N, self_=True, max_split=8):
    """csrc/syrk.hip sy_plan (s0 = 0): tiles, items per split, splits."""
    nt = (T + TILE - 1) // TILE
    ntl = nt * (nt + 1) // 2
    nchunk = N // 64
    nfull = ntl - nt if self_ else ntl
    per_split = nfull + (nt + 1) // 2 if self_ else ntl
    S = max(1, min(max_split, 256 // (nslab * per_split)))
    S = min(S, nchunk)
    return dict(nt=nt, ntl=ntl, nchunk=nchunk, nfull=nfull, per_split=per_split, nsplit=S, ips=per_split * S)


def sy_item(p, T, itx, self_=True):
    """csrc/syrk.hip sy_item: (ta, tb, split, kind) of work item itx of a slab."""
    r, split = itx, 0
    while r >= p["per_split"]:
        r -= p["per_split"]
        split += 1
    if not self_ or r < p["nfull"]:
        t = 0
        while r >= (t if self_ else t + 1):
            r -= t if self_ else t + 1
            t += 1
        return t, r, split, FULL
    ta = 2 * (r - p["nfull"])
    tb = ta + 1 if ta + 1 < p["nt"] else ta
    return ta, tb, split, DIAG1 if tb == ta else DIAG2


def check_scores(B, nh, T, N, strides, numel):
    """Every k_sy_scores workgroup: its item, x rows and columns, partial tiles."""
    nslab = B * nh
    p = sy_plan(nslab, T, N)
    S, ntl = p["nsplit"], p["ntl"]
    grid = 8 * ((nslab + 7) // 8) * p["ips"]
    seen = set()
    chunks_seen = {}
    for bid in range(grid):
        xcd, kk = bid & 7, bid >> 3
        grp = kk // p["ips"]
        slab = grp * 8 + xcd
        if slab >= nslab:
            continue
        ta, tb, split, kind = sy_item(p, T, kk - grp * p["ips"])
        assert split < S
        if kind == FULL:
            assert 0 <= tb < ta < p["nt"]
        else:  # diagonal tiles ta and tb = ta + 1 (or ta alone)
            assert 0 <= ta < p["nt"] and tb == (ta + 1 if kind == DIAG2 else ta) < p["nt"]
        # tiles stored by the item's waves (sy_scores_body: tile_out)
        tiles = [ta * (ta + 1) // 2 + tb] if kind == FULL else [ta * (ta + 1) // 2 + ta] + (
            [tb * (tb + 1) // 2 + tb] if kind == DIAG2 else [])
        for t in tiles:
            assert 0 <= t < ntl
            key = (slab, t, split)
            assert key not in seen, f"tile {key} computed twice"
            seen.add(key)
        # x loads: rows min(tile * 256 + r, T - 1) of both row blocks; stage
        # columns kofs(s) + 8 c + [0, 8) for stages s < 2 nch (later stages
        # re-load the last one).  Split `split` owns the contiguous chunk range
        # [kc0, kc0 + nch) and walks it from chunk krs (set by the slab's group
        # on its XCD): every chunk of the range once per k16 half.
        kc0 = split * p["nchunk"] // S
        nch = (split + 1) * p["nchunk"] // S - kc0
        assert nch >= 1
        krs = ((slab >> 3) * max(1, nch >> 2)) % nch
        cols = [(kc0 + ((s >> 1) + krs) % nch) * 64 + (s & 1) * 32 for s in range(2 * nch)]
        assert sorted(cols) == [kc0 * 64 + 32 * i for i in range(2 * nch)]
        chunks_seen.setdefault((slab, kind), set()).update((c // 64, split) for c in cols)
        max_col = max(cols) + 8 * 3 + 8
        assert max_col <= N
        b, h = divmod(slab, nh)
        max_row = min(max(ta, tb) * TILE + TILE - 1, T - 1)
        hi = b * strides[0] + h * strides[1] + max_row * strides[2] + max_col
        assert hi <= numel
        # partial stores: ((slab ntl + tile) S + split) 65536 + ws NM 1024 + m 1024 + {0, 512} + 8 l + [0, 8)
        for t in tiles:
            nm, nws = (8, 8) if kind == FULL else (9, 4)
            top = ((slab * ntl + t) * S + split) * TILE_ELEMS + (nws - 1) * nm * 1024 + (nm - 1) * 1024 + 512 + 63 * 8 + 8
            assert top <= (slab * ntl + t + 1) * S * TILE_ELEMS
    assert len(seen) == nslab * ntl * S
    # the splits of one slab cover every k chunk, each with exactly one split
    for (slab, kind), cs in chunks_seen.items():
        assert sorted(c for c, _ in cs) == list(range(p["nchunk"])), (slab, kind)
    return p


def sv_grid(nslab, nrb, contiguous=False):
    """csrc/syrk.hip k_sy_sv (slab s on XCD s % 8) and k_sv_dma (XCD x holds slabs
    [x nsx, (x + 1) nsx)): (rb, slab) of each linear workgroup id (None past the slabs)."""
    out = []
    nsx = (nslab + 7) // 8
    for L in range(8 * nsx * nrb):
        xcd, kk = L & 7, L >> 3
        slab = xcd * nsx + kk % nsx if contiguous else (kk % nsx) * 8 + xcd
        out.append(None if slab >= nslab else (nrb - 1 - kk // nsx, slab))
    return out


def check_sv(B, nh, T, D, p, v_strides, v_numel):
    """k_sy_sv: every (row block, slab) workgroup, each 256-column launch."""
    nslab = B * nh
    nrb = (T + 63) // 64
    S, ntl = p["nsplit"], p["ntl"]
    part_elems = nslab * ntl * S * TILE_ELEMS
    # the 1-D grid visits each (row block, slab) once; slab s sits on XCD s % 8
    # (k_sy_sv) or XCD s / nsx (k_sv_dma), row blocks longest first
    nsx = (nslab + 7) // 8
    for contiguous in (False, True):
        grid = sv_grid(nslab, nrb, contiguous)
        live = [g for g in grid if g is not None]
        assert sorted(live) == sorted((rb, s) for s in range(nslab) for rb in range(nrb))
        assert all((g[1] // nsx if contiguous else g[1] % 8) == L % 8 for L, g in enumerate(grid) if g is not None)
    grid = sv_grid(nslab, nrb)
    # on each XCD the row blocks (rb + 1 key chunks each) start longest first
    for x in range(8):
        rbs = [g[0] for L, g in enumerate(grid) if L % 8 == x and g is not None]
        assert rbs == sorted(rbs, reverse=True)
    for d0 in range(0, D, 256):
        Dc = min(256, D - d0)
        assert Dc % 8 == 0
        for rb in range(nrb):
            r0 = rb * 64
            nch = (min(T, r0 + 64) + 63) // 64
            ti = r0 >> 8
            for ck in range(nch):
                tj = (ck * 64) >> 8
                assert tj <= ti
                tile = ti * (ti + 1) // 2 + tj
                # the piece read for split sp: slot (< 64 full, < 36 diagonal) * 1024 + half * 512 + 8 l + [0, 8)
                top = ((nslab - 1) * ntl + tile) * S * TILE_ELEMS + (S - 1) * TILE_ELEMS + 63 * 1024 + 512 + 63 * 8 + 8
                assert top <= part_elems
            # V rows min(j, T - 1) of chunks < nch, columns 8 min(vc, Dc / 8 - 1) + [0, 8) of the launch's slice
            max_v = (B - 1) * v_strides[0] + (T - 1) * v_strides[2] + d0 + 8 * (Dc // 8 - 1) + 8
            assert max_v <= v_numel


def check_decode(B, nh, S, N, D, cap):
    """k_decode_bf16 over capacity-strided past views (KVCache.past: rows [0, S) of (B, nh, cap, N))."""
    assert N % 2048 == 0  # the kernel's 16-byte pieces: nc = N / 512, c += 4
    k_strides = (nh * cap * N, cap * N, N)
    v_strides = (cap * D, 0, D)
    nred = (S + 63) // 64
    rows = B * nh
    for chunk in range(nred):
        s0, s1 = chunk * 64, min(S, chunk * 64 + 64)
        assert s0 < s1
        # keys s0 + wave + 8 j (and + 4 when < s1): all < s1 <= S
        keys = [s for wave in range(4) for s in range(s0 + wave, s1, 8)]
        keys += [s + 4 for s in keys if s + 4 < s1]
        assert max(keys) < S and min(keys) >= 0
        nc = N // 512
        max_col = 63 * 8 + (nc - 1) * 512 + 8
        assert max_col <= N
        hi = (B - 1) * k_strides[0] + (nh - 1) * k_strides[1] + (S - 1) * k_strides[2] + max_col
        assert hi <= B * nh * cap * N  # inside the layer's cache block
        assert (B - 1) * v_strides[0] + (S - 1) * v_strides[2] + D <= B * cap * D
    assert nred * rows * D > 0


@pytest.mark.parametrize("name,B,nh,T,N,D", PREFILL, ids=[c[0] for c in PREFILL])
def test_prefill_launches_stay_in_bounds(name, B, nh, T, N, D):
    # x_sparse: the permuted (B, T, nh, N) encoder output viewed as (B, nh, T, N)
    x_strides = (T * nh * N, N, nh * N)
    p = check_scores(B, nh, T, N, x_strides, B * T * nh * N)
    # V: the layer input (B, 1, T, D), contiguous
    check_sv(B, nh, T, D, p, (T * D, 0, D), B * T * D)


@pytest.mark.parametrize("S", [256, 257, 300, 383, 384, 448, 511])
def test_decode_launches_stay_in_bounds(S):
    # C3 generate: B = 64, nh = 4, N = 8192, D = 256, cache capacity prompt + new = 512
    check_decode(64, 4, S, 8192, 256, 512)


def test_restated_plan_matches_the_documented_c1_split():
    # C1: 32 slabs, one full tile + one diagonal pair per split, 4 splits = 256 items
    p = sy_plan(32, 512, 8192)
    assert (p["per_split"], p["nsplit"], p["ips"]) == (2, 4, 8)
    assert 8 * ((32 + 7) // 8) * p["ips"] == 256
    # every item kind appears, pairs cover both diagonal tiles
    kinds = {sy_item(p, 512, i)[3] for i in range(p["ips"])}
    assert kinds == {FULL, DIAG2}
    assert {sy_item(p, 512, i)[:2] for i in range(p["ips"])} == {(1, 0), (0, 1)}


def test_a_planted_overrun_is_caught():
    # the checker itself: a row stride one element too long overruns the buffer
    B, nh, T, N = 2, 4, 300, 512
    with pytest.raises(AssertionError):
        check_scores(B, nh, T, N, (T * nh * N, N, nh * N + 1), B * T * nh * N)
    check_scores(B, nh, T, N, (T * nh * N, N, nh * N), B * T * nh * N)


def check_dq_rot(B, nh, T, N, x_strides, x_numel, tpad):
    """csrc/syrk.hip k_dq_sy with the B rotation, on x itself: B chunk u of lane (w, lane)
    is row min(32 st + brow, T - 1), brow = 2 (8 u + w) + lane / 32, columns n0 + 8 (pb ^ 4 (brow & 3))
    + [0, 8), pb = lane % 32; its frequencies at element (n0 + 8 (...)) + 2 j + [0, 1], j < 4."""
    ntn = N // TILE
    nst = tpad // 32
    for b, h in ((0, 0), (B - 1, nh - 1)):
        for tn in (0, ntn - 1):
            n0 = tn * TILE
            for st in (0, nst - 1):
                for u in (0, 1):
                    for w in (0, 7):
                        for lane in (0, 31, 32, 63):
                            brow = 2 * (8 * u + w) + lane // 32
                            row = min(32 * st + brow, T - 1)
                            col = n0 + 8 * ((lane % 32) ^ (4 * (brow & 3)))
                            assert col + 8 <= N and col + 2 * 3 + 1 < N
                            assert b * x_strides[0] + h * x_strides[1] + row * x_strides[2] + col + 8 <= x_numel
                            # the byte offset within the slab fits the DMA's 32-bit voffset
                            assert (row * x_strides[2] + col) * 2 < 2 ** 32


def check_dv(B, nh, Hv, T, N, D, p):
    """csrc/syrk.hip k_dv_sy: 1-D grid of 8 per_xcd workgroups, workgroup L the unit
    u = (L % 8) per_xcd + L / 8 = bv nrb + rb (units past nrb B Hv return), every unit
    taken once; two groups taking items g, g + 2, ... of (64-row chunk nrb - 1 - it / nhv
    >= rb, head h_lo + it % nhv); loads of item min(it, total - 1); M pieces of tile
    (ti, tj), ti >= tj, splits < nsplit; dO rows < T (others zero); dV rows < T."""
    nrb = (T + 63) // 64
    nbv = B * Hv
    per_xcd = (nrb * nbv + 7) // 8
    units = [(L % 8) * per_xcd + L // 8 for L in range(8 * per_xcd)]
    units = [u for u in units if u < nrb * nbv]
    assert sorted(units) == list(range(nrb * nbv))
    S, ntl = p["nsplit"], p["ntl"]
    part_elems = B * nh * ntl * S * TILE_ELEMS
    for u in units:
        bv, rb = divmod(u, nrb)
        b, hv = divmod(bv, Hv)
        h_lo, h_hi = (0, nh) if Hv == 1 else (hv, hv + 1)
        nhv = h_hi - h_lo
        total = (nrb - rb) * nhv
        assert total >= 1
        seen = set()
        for grp in (0, 1):
            nk = (total + 1) // 2
            for k in range(nk + 1):  # steps plus the load issued after the last one
                it = min(grp + 2 * k, total - 1)
                ic = nrb - 1 - it // nhv
                h = h_lo + it - (nrb - 1 - ic) * nhv
                assert h_lo <= h < h_hi and rb <= ic < nrb
                if grp + 2 * k < total:
                    seen.add((h, ic))
                ti, tj = (ic * 64) >> 8, (rb * 64) >> 8
                assert tj <= ti
                slab = b * nh + h
                tile = ti * (ti + 1) // 2 + tj
                top = ((slab * ntl + tile) * S + S - 1) * TILE_ELEMS + 63 * 1024 + 512 + 63 * 8 + 8
                assert top <= part_elems
        assert seen == {(h, ic) for h in range(h_lo, h_hi) for ic in range(rb, nrb)}


DV_STAGE, DV_RING, DV_PITCH = 8192 + 64 * 512, 3, 1056


def check_dv_dma(B, nh, Hv, T, N, D, p, d_strides, d_numel):
    """csrc/syrk.hip k_dv_dma (one split): the units and items of k_dv_sy; per item
    wave w moves half w & 1 of M block (w >> 2, (w >> 1) & 1) (one 1 KB DMA inside its
    tile) and dO rows 8 w + 2 v + lane / 32, clamped to T - 1, chunk (lane % 32) ^
    4 (row & 3) clamped to D / 8 - 1, into stage slot (item % 3) of the 120 KB ring;
    fragment reads and the 64 x 1056-byte output tile stay in the ring; the A operand's
    rows (16 hf + 8 (t / 4) + 4 (l / 32) + t % 4) are the stored accumulator rows."""
    assert p["nsplit"] == 1
    nrb = (T + 63) // 64
    nbv = B * Hv
    per_xcd = (nrb * nbv + 7) // 8
    units = sorted(u for u in ((L % 8) * per_xcd + L // 8 for L in range(8 * per_xcd)) if u < nrb * nbv)
    assert units == list(range(nrb * nbv))
    ntl = p["ntl"]
    part_bytes = B * nh * ntl * TILE_ELEMS * 2
    lane = np.arange(64)
    for u in units:
        bv, rb = divmod(u, nrb)
        b, hv = divmod(bv, Hv)
        h_lo, nhv = (0, nh) if Hv == 1 else (hv, 1)
        total = (nrb - rb) * nhv
        for it in range(total):
            c = it // nhv
            ic, h = nrb - 1 - c, h_lo + it - c * nhv
            assert rb <= ic < nrb
            ti, tj = (ic * 64) >> 8, (rb * 64) >> 8
            assert tj <= ti
            tile = ((b * nh + h) * ntl + ti * (ti + 1) // 2 + tj) * TILE_ELEMS * 2
            # slot index < 64, half < 2: the 1 KB piece ends inside the tile
            assert tile + 63 * 2048 + 1024 + 63 * 16 + 16 <= part_bytes
            slot = it % DV_RING
            for w in range(8):
                assert slot * DV_STAGE + w * 1024 + 1024 <= slot * DV_STAGE + 8192
                for v in range(4):
                    r = 8 * w + 2 * v + lane // 32
                    row = np.minimum(ic * 64 + r, T - 1)
                    cc = np.minimum((lane % 32) ^ (4 * (r & 3)), D // 8 - 1)
                    off = row * d_strides[2] + 8 * cc
                    assert int((b * d_strides[0] + h * d_strides[1] + off + 8).max()) <= d_numel
                    assert int((off * 2 + 16).max()) < 2 ** 32
                    assert slot * DV_STAGE + 8192 + 4096 * w + 1024 * v + 64 * 16 <= (slot + 1) * DV_STAGE
    # fragment reads inside a stage: A halves, B transposing reads (row 4 g + q / 4, 8 below)
    for w in range(8):
        kq, wc = w >> 2, w & 3
        for hf in (0, 1):
            ks = 2 * kq + hf
            for jb in (0, 1):
                assert ((2 * kq + jb) * 2 + hf) * 1024 + 63 * 16 + 16 <= 8192
            for c in (0, 1):
                g4, q = lane >> 4, lane & 15
                row = 4 * (g4 >> 1) + (q >> 2)
                col = 64 * wc + 32 * c + 16 * (g4 & 1) + 4 * (q & 3)
                boff = 8192 + row * 512 + (((col >> 3) ^ (4 * (row & 3))) * 16) + ((col >> 2) & 1) * 8
                assert int((boff + ks * 16 * 512 + 8 * 512 + 8).max()) <= DV_STAGE
                # the B rows of lane l, value t are the A rows of the same (l / 32, t)
                for t in range(8):
                    brow = 16 * ks + 4 * (lane >> 5) + 8 * (t >> 2) + (t & 3)
                    arow = 32 * kq + 16 * hf + 8 * (t >> 2) + 4 * (lane >> 5) + (t & 3)
                    assert (brow == arow).all()
    # the stored accumulator rows of value t = 2 qq + e of half hf, lane l
    for l in range(64):
        for hf in (0, 1):
            for t in range(8):
                r = 2 * (4 * hf + t // 2) + t % 2
                stored = 8 * (r >> 2) + 4 * (l >> 5) + (r & 3)
                assert stored == 16 * hf + 8 * (t >> 2) + 4 * (l >> 5) + (t & 3)
    assert 64 * DV_PITCH <= DV_RING * DV_STAGE and DV_PITCH % 16 == 0


def check_sv_dma(B, nh, Hv, T, N, D, p, v_strides, v_numel):
    """csrc/syrk.hip k_sv_dma (one split, bf16 V): the k_sy_sv grid; per key chunk wave w
    moves half w & 1 of M block (w >> 2, (w >> 1) & 1) (DMA lane l loads stored lane
    l ^ 4 (l / 32) ^ 8 hf, a permutation of the 64) and V rows 8 w + 2 v + lane / 32
    (clamped to T - 1, chunk (lane % 32) ^ 4 (row & 3) clamped to Dc / 8 - 1) into stage
    (chunk % 3) of the 120 KB ring; the transposing A reads find, for every lane and key,
    the stored element (row i, key j) in its LDS slot; B reads and the output tile stay
    in the ring."""
    assert p["nsplit"] == 1
    nslab = B * nh
    nrb = (T + 63) // 64
    ntl = p["ntl"]
    part_bytes = nslab * ntl * TILE_ELEMS * 2
    lane = np.arange(64)
    for hf in (0, 1):
        perm = lane ^ (4 * (lane >> 5)) ^ (8 * hf)
        assert sorted(perm) == list(range(64))
    # element (i, j) of a stored 32 x 32 block: half i >> 4, stored lane j + 32 ((i >> 2) & 1),
    # value 4 ((i >> 3) & 1) + (i & 3); LDS slot of stored lane L' in half hf: L' ^ 4 (L' >> 5) ^ 8 hf
    def lds_byte(i, j):
        hf = i >> 4
        lp = j + 32 * ((i >> 2) & 1)
        slot = lp ^ (4 * (lp >> 5)) ^ (8 * hf)
        return hf * 1024 + slot * 16 + 2 * (4 * ((i >> 3) & 1) + (i & 3))
    # ds_read_b64_tr_b16 within a group of 16 lanes: result lane q, value e is element q & 3
    # of the 8 bytes read by lane 4 e + q / 4
    for k2 in (0, 1):
        for r in (0, 1):
            for l in range(64):
                g4, q = l >> 4, l & 15
                for e in range(4):
                    s = 4 * e + (q >> 2)
                    sl = 16 * k2 + 8 * (g4 >> 1) + 4 * r + (s >> 2) + 32 * (s & 1)
                    slot = sl ^ (4 * (sl >> 5)) ^ (8 * (g4 & 1))
                    addr = (g4 & 1) * 1024 + slot * 16 + 8 * ((s >> 1) & 1) + 2 * (q & 3)
                    i = 16 * (g4 & 1) + q
                    j = 16 * k2 + 8 * (g4 >> 1) + 4 * r + e
                    assert addr == lds_byte(i, j), (k2, r, l, e)
    for d0 in range(0, D, 256):
        Dc = min(256, D - d0)
        for slab in sorted({0, nslab - 1}):  # the V base of the first and last slab
            b, h = divmod(slab, nh)
            hv = 0 if Hv == 1 else h
            for rb in range(nrb):
                r0 = rb * 64
                nch = (min(T, r0 + 64) + 63) // 64
                ti = r0 >> 8
                for ck in range(nch):
                    tj = (ck * 64) >> 8
                    assert tj <= ti
                    tile = (slab * ntl + ti * (ti + 1) // 2 + tj) * TILE_ELEMS * 2
                    assert tile + 63 * 2048 + 1024 + 63 * 16 + 16 <= part_bytes
                    slot = ck % DV_RING
                    for w in range(8):
                        for v in range(4):
                            rr = 8 * w + 2 * v + lane // 32
                            row = np.minimum(ck * 64 + rr, T - 1)
                            cc = np.minimum((lane % 32) ^ (4 * (rr & 3)), Dc // 8 - 1)
                            off = row * v_strides[2] + d0 + 8 * cc
                            assert int((b * v_strides[0] + hv * v_strides[1] + off + 8).max()) <= v_numel
                            assert int(((row * v_strides[2] + 8 * cc) * 2 + 16).max()) < 2 ** 32
                            assert slot * DV_STAGE + 8192 + 4096 * w + 1024 * v + 64 * 16 <= (slot + 1) * DV_STAGE
    for w in range(8):
        kh, wc = w >> 2, w & 3
        for k2 in (0, 1):
            ks = 2 * kh + k2
            for c in (0, 1):
                g4, q = lane >> 4, lane & 15
                row = 8 * (g4 >> 1) + (q >> 2)
                col = 64 * wc + 32 * c + 16 * (g4 & 1) + 4 * (q & 3)
                boff = 8192 + row * 512 + (((col >> 3) ^ (4 * (row & 3))) * 16) + ((col >> 2) & 1) * 8
                assert int((boff + ks * 16 * 512 + 4 * 512 + 8).max()) <= DV_STAGE
            for ib in (0, 1):
                assert ib * 4096 + kh * 2048 + 1024 + 63 * 16 + 16 <= 8192


@pytest.mark.parametrize("B,nh,Hv,T,N,D", [(16, 4, 1, 1024, 256, 256), (8, 4, 1, 1000, 256, 192), (8, 4, 4, 700, 256, 64),
                                            (130, 1, 1, 33, 256, 128), (8, 4, 1, 520, 256, 512)])
def test_sv_ring_launches_stay_in_bounds(B, nh, Hv, T, N, D):
    p = sy_plan(B * nh, T, N)
    check_sv_dma(B, nh, Hv, T, N, D, p, (Hv * T * D, T * D, D), B * Hv * T * D)


@pytest.mark.parametrize("B,nh,Hv,T,N,D", [(16, 4, 1, 1024, 256, 256), (8, 4, 1, 1000, 256, 192), (8, 4, 4, 700, 256, 64),
                                            (130, 1, 1, 33, 256, 128), (32, 4, 1, 512, 8192, 256)])
def test_dv_ring_launches_stay_in_bounds(B, nh, Hv, T, N, D):
    p = sy_plan(B * nh, T, N)
    check_dv_dma(B, nh, Hv, T, N, D, p, (nh * T * D, T * D, D), B * nh * T * D)


@pytest.mark.parametrize("B,nh,T,N,D", [(32, 4, 512, 8192, 256), (3, 2, 300, 512, 64), (1, 3, 700, 768, 256)])
def test_rope_backward_launches_stay_in_bounds(B, nh, T, N, D):
    # the training backward from kept tiles: x_sparse as the permuted (B, T, nh, N) view
    tpad = ((T + 63) // 64) * 64
    check_dq_rot(B, nh, T, N, (T * nh * N, N, nh * N), B * T * nh * N, tpad)
    p = sy_plan(B * nh, T, N)
    check_dv(B, nh, 1, T, N, D, p)
    check_dv(B, nh, nh, T, N, D, p)


def check_gated(B, T, nh, N, K):
    """csrc/model.hip k_gated_gemm on contiguous y (B, nh, T, K), wt (nh, N, K) and x (B, T, nh, N):
    every tile's DMA chunks (instruction u of wave w, lane l: A row 16 (8u + w) + l / 4, u < 2, or
    B row 16 w + l / 4, u = 2; chunk (l & 3) ^ ((l >> 4) & 3); stage s adds 32 s elements) and
    epilogue x chunks (row (tid >> 4) + 32 e, columns n0 + 8 (tid & 15), clamped) stay inside their
    views, the DMA byte offsets fit 32 bits, and the LDS bytes a stage fills stay inside the
    3-slot ring of 24 KB slots."""
    GM, GN, GK, STAGE, RING = 256, 128, 32, 24 * 1024, 3
    M = B * T
    y0, y2 = nh * T * K, K
    nst = K // GK
    nmb, nnb = (M + GM - 1) // GM, (N + GN - 1) // GN
    y_head, w_head = B * nh * T * K - (nh - 1) * T * K, N * K  # elements reachable from a head's base
    for mbi in {0, nmb - 1}:
        for nbi in {0, nnb - 1}:
            m0, n0 = mbi * GM, nbi * GN
            for w in (0, 7):
                for lane in (0, 3, 16, 63):
                    dc = (lane & 3) ^ ((lane >> 4) & 3)
                    for u in (0, 1):
                        m = min(m0 + 16 * (8 * u + w) + lane // 4, M - 1)
                        b, tt = divmod(m, T)
                        off = b * y0 + tt * y2 + dc * 8
                        last = off + 32 * (nst - 1) + 8
                        assert last <= y_head and off * 2 < 2 ** 32 and (last - 8) * 2 < 2 ** 32
                        assert ((nst - 1) % RING) * STAGE + (8 * u + w) * 1024 + lane * 16 + 16 <= RING * STAGE
                    n = min(n0 + 16 * w + lane // 4, N - 1)
                    off = n * K + dc * 8
                    assert off + 32 * (nst - 1) + 8 <= w_head and (off + 32 * (nst - 1)) * 2 < 2 ** 32
                    assert 2 * STAGE + 16 * 1024 + w * 1024 + lane * 16 + 16 <= RING * STAGE
            for tid in (0, 15, 496, 511):
                for e in range(8):
                    m = min(m0 + (tid >> 4) + 32 * e, M - 1)
                    b, tt = divmod(m, T)
                    col = min(n0 + 8 * (tid & 15), N - 8)
                    assert b * T * nh * N + tt * nh * N + (nh - 1) * N + col + 8 <= B * T * nh * N


@pytest.mark.parametrize("B,T,nh,N,K", [(32, 512, 4, 8192, 256), (4, 2048, 8, 8192, 512), (2, 300, 2, 1000, 96),
                                       (3, 257, 3, 136, 64), (1, 1, 1, 8, 32)])
def test_gated_gemm_launches_stay_in_bounds(B, T, nh, N, K):
    check_gated(B, T, nh, N, K)


def check_gated_dec(B, T, nh, N):
    """csrc/gated_dec.hip k_gated_dec + k_head_sum on the harness's contiguous operands y (B, nh, T,
    256), wt (nh, N, 256), x (B, T, nh, N), dec (nh N, 256): the XCD-major grid covers each (head,
    256-token block) once; the LDS-DMA sources of every chunk (encoder_v rows 2i + l / 32 chunk
    (l % 32) ^ (row % 32); decoder rows 2 (i - 16) + l / 32 chunk (l % 32) ^ 4 (row % 4); x rows
    16 (i - 32) + l / 4 chunk (l % 4) ^ ((row / 4) % 4), token clamped to M - 1) stay inside their
    views with 32-bit offsets from the head's base; instruction i of a slot writes LDS bytes
    [i KB + 16 l, +16) inside its 48 KB slot of the 3-slot ring; the fragment reads (encoder_v
    row l % 32 chunk (2s + l / 32) ^ (l % 32); decoder transposing reads at 16 k2 + 4 (g4 / 2) +
    q / 4 (+ 8) rows; x pieces) stay inside the region of the slot they read; the y loads, the
    partial stores [h][m][256] (m < M) and k_head_sum's reads stay in bounds."""
    K = D = MT = 256
    NC, SLOT, RING = 32, 48 * 1024, 3
    WV, DEC = NC * K * 2, NC * D * 2
    M = B * T
    ntb = (M + MT - 1) // MT
    total = ntb * nh
    per_xcd = (total + 7) // 8
    seen = []
    for bid in range(8 * per_xcd):
        xcd, kk0 = bid & 7, bid >> 3
        t = xcd * per_xcd + kk0
        if t < total:
            seen.append(divmod(t, ntb))
    assert sorted(seen) == [(h, tb) for h in range(nh) for tb in range(ntb)]
    assert RING * SLOT <= 160 * 1024
    nck = N // NC
    part_elems = nh * M * D
    for h in {0, nh - 1}:
        for tb in {0, ntb - 1}:
            m0 = tb * MT
            for w in range(4):
                for lane in (0, 5, 31, 32, 47, 63):
                    hl, l32 = lane >> 5, lane & 31
                    for u in range(12):
                        i = 4 * u + w
                        for slot in range(RING):
                            lds = slot * SLOT + u * 4096 + w * 1024 + 16 * lane
                            assert slot * SLOT + i * 1024 <= lds and lds + 16 <= slot * SLOT + (i + 1) * 1024
                            assert lds + 16 <= (slot + 1) * SLOT
                        for ck in (0, nck - 1, nck, nck + 1):  # issue(ck + 2) past the end re-loads the last chunk
                            cc = min(ck, nck - 1)
                            if i < 16:
                                r = 2 * i + hl
                                c = l32 ^ (r & 31)
                                assert 0 <= r < NC and 0 <= c < 32
                                off = (cc * NC + r) * K + 8 * c  # from the head's base (wt + h N K)
                                assert off * 2 < 2 ** 32 and h * N * K + off + 8 <= nh * N * K
                            elif i < 32:
                                r = 2 * (i - 16) + hl
                                c = l32 ^ (4 * (r & 3))
                                assert 0 <= c < 32
                                off = (cc * NC + r) * D + 8 * c
                                assert off * 2 < 2 ** 32 and h * N * D + off + 8 <= nh * N * D
                            else:
                                r = 16 * (i - 32) + (lane >> 2)
                                c = (lane & 3) ^ ((r >> 2) & 3)
                                assert 0 <= r < MT and 0 <= c < 4
                                m = min(m0 + r, M - 1)
                                b, tt = divmod(m, T)
                                e = b * T * nh * N + tt * nh * N + h * N + 8 * c + cc * NC
                                assert e + 8 <= B * T * nh * N and 8 * c + cc * NC + 8 <= N
                    for j in range(2):
                        m = min(m0 + 64 * w + 32 * j + l32, M - 1)
                        b, tt = divmod(m, T)
                        yo = b * nh * T * K + h * T * K + tt * K + 8 * hl
                        assert yo + 16 * 15 + 8 <= B * nh * T * K
                    # the kernel forms these addresses as a per-lane base XOR a compile-time offset
                    wvb = l32 * 512 + 16 * (hl ^ (l32 & 1)) + 32 * (l32 >> 1)
                    for s in range(16):
                        o = l32 * 512 + 16 * ((2 * s + hl) ^ l32)
                        assert o == wvb ^ (32 * s)
                        assert 0 <= o and o + 16 <= WV
                    g4, q = lane >> 4, lane & 15
                    drow = 4 * (g4 >> 1) + (q >> 2)
                    dvb = WV + drow * 512 + 32 * (g4 & 1) + 16 * ((q & 3) >> 1) + 8 * (q & 1) + 64 * (drow & 3)
                    for db in range(8):
                        col = 32 * db + 16 * (g4 & 1) + 4 * (q & 3)
                        o = WV + drow * 512 + (((col >> 3) ^ (4 * (drow & 3))) * 16) + ((col >> 2) & 1) * 8
                        assert o == dvb ^ (64 * db)
                        for k2 in range(2):
                            for extra in (0, 8 * 512):
                                p = o + k2 * 16 * 512 + extra
                                assert WV <= p and p + 8 <= WV + DEC
                    xvb = WV + DEC + (64 * w + l32) * 64 + 8 * hl + 16 * ((l32 >> 2) & 3)
                    for j in range(2):
                        r = 64 * w + 32 * j + l32
                        for p in range(4):
                            o = WV + DEC + r * 64 + 16 * (p ^ ((r >> 2) & 3)) + 8 * hl
                            assert o == (xvb + 2048 * j) ^ (16 * p)
                            assert WV + DEC <= o and o + 8 <= SLOT
                        for rr in range(16):
                            m = m0 + 64 * w + 32 * j + 8 * (rr >> 2) + 4 * hl + (rr & 3)
                            if m < M:
                                for db in range(8):
                                    assert (h * M + m) * D + 32 * db + l32 < part_elems
    nthr = (M * D // 4 + 255) // 256
    for e in {0, (nthr * 256 - 1) * 4, (M * D // 4 - 1) * 4}:
        if e < M * D:
            assert (nh - 1) * M * D + e + 4 <= part_elems


@pytest.mark.parametrize("B,T,nh,N", [(32, 512, 4, 8192), (64, 256, 4, 8192), (2, 300, 2, 1024), (3, 129, 4, 96),
                                      (1, 257, 1, 32)])
def test_gated_decoder_launches_stay_in_bounds(B, T, nh, N):
    check_gated_dec(B, T, nh, N)


def check_relu_enc(B, T, nh, N, K):
    """csrc/enc.hip k_relu_enc on the harness's operands y (B, 1, T, K) expanded over the heads
    (head stride 0), wt (nh, N, K), out (B, T, nh, N): the XCD-major grid covers each (head,
    256-token block) once; each chunk's DMA (instruction i = 4 u + w: K = 256 rows 2 i + l / 32,
    position l % 32; K = 512 row i, position l; chunk position ^ (row % 32)) reads inside wt with
    32-bit offsets from the head's base and writes its 1 KB of the 32 KB slot; the fragment
    reads stay in their slot; the tile writes and reads stay in their tile; the gated form's x
    DMA writes its tile bytes, only rows the same wave reads, from inside x; the y loads and the
    output stores (the chunk walk wraps from the block's starting chunk) stay in bounds."""
    MT, SLOT, RING = 256, 32 * 1024, 3
    NC = 64 if K == 256 else 32
    ROWB, NB, KS = K * 2, NC // 32, K // 16
    TROW = NC * 2
    TILE, TCH = MT * TROW, TROW // 16
    SPT, RSTEP = MT * TCH // 256, 256 // TCH
    assert RING * SLOT + 2 * TILE <= 160 * 1024 and N % NC == 0
    M = B * T
    ntb = (M + MT - 1) // MT
    total = ntb * nh
    per_xcd = (total + 7) // 8
    seen = []
    for bid in range(8 * per_xcd):
        t = (bid & 7) * per_xcd + (bid >> 3)
        if (bid >> 3) < per_xcd and t < total:
            seen.append(divmod(t, ntb))
    assert sorted(seen) == [(h, tb) for h in range(nh) for tb in range(ntb)]
    nck = N // NC
    assert (N - 1) * K * 2 + K * 2 < 2 ** 32
    for h in {0, nh - 1}:
        for tb in {0, ntb - 1}:
            m0 = tb * MT
            c0 = tb * nck // ntb % nck
            chunks = {(c + c0) % nck for c in (0, nck - 1)} | {nck - 1}
            for w in range(4):
                for lane in (0, 7, 31, 32, 63):
                    hl, l32 = lane >> 5, lane & 31
                    for u in range(8):
                        i = 4 * u + w
                        r = 2 * i + hl if K == 256 else i
                        p = l32 if K == 256 else lane
                        c = p ^ (r & 31)
                        assert 0 <= r < NC and 0 <= c < K // 8
                        for slot in range(RING):
                            lds = slot * SLOT + u * 4096 + w * 1024 + 16 * lane
                            assert lds == slot * SLOT + i * 1024 + 16 * lane and lds + 16 <= (slot + 1) * SLOT
                        for cc in chunks:
                            off = (cc * NC + r) * K + 8 * c
                            assert off * 2 < 2 ** 32 and h * N * K + off + 8 <= nh * N * K
                    for j in range(2):
                        m = min(m0 + 64 * w + 32 * j + l32, M - 1)
                        b, tt = divmod(m, T)
                        assert b * T * K + tt * K + 8 * hl + 16 * (KS - 1) + 8 <= B * T * K
                    for s_ in range(KS):
                        for i in range(NB):
                            o = i * 32 * ROWB + l32 * ROWB + 16 * ((2 * s_ + hl) ^ l32)
                            assert 0 <= o and o + 16 <= SLOT
                    for it in range(NB * 8):
                        i, j, q = it // 8, (it // 4) & 1, it & 3
                        row = 64 * w + 32 * j + l32
                        o = row * TROW + 16 * ((4 * i + q) ^ (row & (TCH - 1))) + 8 * hl
                        assert 0 <= o and o + 8 <= TILE
            # gated form: x pieces by LDS DMA into the tile, instruction u of wave w
            # rows RPI (4 u + w) + l / TCH: the same rows as the wave's own tile reads
            RPI, XI = 1024 // TROW, TILE // 1024 // 4
            for w in range(4):
                dma_rows = {RPI * (4 * u + w) + lane // TCH for u in range(XI) for lane in range(64)}
                read_rows = {(64 * w + lane) // TCH + RSTEP * e for lane in range(64) for e in range(SPT)}
                assert dma_rows == read_rows
                for u in range(XI):
                    for lane in (0, 3, 31, 63):
                        r = RPI * (4 * u + w) + lane // TCH
                        piece = (lane % TCH) ^ (r & (TCH - 1))
                        lds = (4 * u + w) * 1024 + 16 * lane
                        assert lds + 16 <= TILE and lds == r * TROW + 16 * (lane % TCH)
                        m = min(m0 + r, M - 1)
                        b, tt = divmod(m, T)
                        for cc in chunks:
                            o = b * T * nh * N + tt * nh * N + h * N + 8 * piece + cc * NC
                            assert o + 8 <= B * T * nh * N and 8 * piece + cc * NC + 8 <= N
            for tid in (0, 5, 100, 255):
                spc = tid % TCH
                for e in range(SPT):
                    r = tid // TCH + RSTEP * e
                    assert r < MT and r * TROW + 16 * (spc ^ (r & (TCH - 1))) + 16 <= TILE
                    m = m0 + r
                    if m < M:
                        b, tt = divmod(m, T)
                        for cc in chunks:
                            o = b * T * nh * N + tt * nh * N + h * N + 8 * spc + cc * NC
                            assert o + 8 <= B * T * nh * N and 8 * spc + cc * NC + 8 <= N


@pytest.mark.parametrize("B,T,nh,N,K", [(32, 512, 4, 8192, 256), (4, 2048, 8, 8192, 512), (64, 256, 4, 8192, 256),
                                        (2, 300, 4, 1024, 256), (3, 129, 3, 192, 512), (1, 1, 2, 64, 256)])
def test_relu_encoder_launches_stay_in_bounds(B, T, nh, N, K):
    check_relu_enc(B, T, nh, N, K)
