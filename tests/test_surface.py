"""CPU tests of the host side: C-ABI library load/exports/validation, the
``kernels`` dispatch surface (reference contracts), eager paths vs the oracle,
golden fixtures, and the bench/entry-point contracts.  No GPU compute."""

from __future__ import annotations

import ctypes
import json
import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "bdh_hip.h"
GOLDEN = Path(__file__).resolve().parent / "golden"


# ------------------------------------------------------------ C-ABI library
def _declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bdh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import bdh_hip_ext as ext

    lib = ctypes.CDLL(ext.lib_path)
    declared = _declared_symbols()
    assert len(declared) >= 14
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert set(declared) == set(ext.EXPORTED_SYMBOLS)


def test_library_host_queries_without_gpu():
    import bdh_hip_ext as ext

    lib = ext._lib
    assert "gfx950" in ext.version()
    assert lib.bdh_error_string(0) == b"ok"
    assert b"shape" in lib.bdh_error_string(1)
    # workspace for the C1 shape: split-K partial score tiles (32 slabs x 3
    # tiles x 4 splits x 256 x 256 bf16) and the score x V part slots
    ws = lib.bdh_tril_score_v_workspace(8, 4, 512, 8192, 256, ext.BDH_BF16)
    assert ws >= 32 * 3 * 4 * 256 * 256 * 2
    assert lib.bdh_tril_decode_workspace(64, 4, 1, 0, 8192, 256) == 64 * 4 * 256 * 4


def _t4(shape, dtype=0, data=0x1000):
    t = __import__("bdh_hip_ext").Tensor4()
    t.data = data
    st = [1, 1, 1, 1]
    for i in (2, 1, 0):
        st[i] = st[i + 1] * shape[i + 1]
    for i in range(4):
        t.size[i] = shape[i]
        t.stride[i] = st[i]
    t.dtype = dtype
    return t


def test_c_abi_rejects_bad_arguments_before_launching():
    """Validation happens on the host; nothing is launched (no GPU needed)."""
    import bdh_hip_ext as ext

    lib = ext._lib
    q = _t4((1, 2, 4, 8))
    v_bad = _t4((1, 3, 4, 5), data=0x9000)  # heads neither 1 nor H
    out = _t4((1, 2, 4, 5), data=0x20000)
    assert lib.bdh_tril_score_v(ctypes.byref(q), ctypes.byref(q), ctypes.byref(v_bad), ctypes.byref(out), None, 0, None) == 1
    v = _t4((1, 1, 4, 5), data=0x9000)
    bad_dtype = _t4((1, 2, 4, 5), dtype=7, data=0x20000)
    assert lib.bdh_tril_score_v(ctypes.byref(q), ctypes.byref(q), ctypes.byref(v), ctypes.byref(bad_dtype), None, 0, None) == 2
    strided = _t4((1, 2, 4, 8))
    strided.stride[3] = 2
    assert lib.bdh_tril_score_v(ctypes.byref(strided), ctypes.byref(strided), ctypes.byref(v), ctypes.byref(out), None, 0, None) == 3
    # output overlapping an input
    alias = _t4((1, 2, 4, 5), data=0x1000)
    assert lib.bdh_tril_score_v(ctypes.byref(q), ctypes.byref(q), ctypes.byref(v), ctypes.byref(alias), None, 0, None) == 7
    # missing workspace
    assert lib.bdh_tril_score_v(ctypes.byref(q), ctypes.byref(q), ctypes.byref(v), ctypes.byref(out), None, 0, None) == 4
    # odd RoPE dim
    x = _t4((1, 2, 4, 7))
    fr = (ctypes.c_float * 7)()
    assert lib.bdh_tril_rope_score_v(ctypes.byref(x), ctypes.byref(v), ctypes.byref(out), fr, 0, None, None, 0, None) == 1
    # decode: k_past heads mismatch
    kp = _t4((1, 3, 6, 8), data=0x40000)
    vp = _t4((1, 1, 6, 5), data=0x80000)
    o1 = _t4((1, 2, 1, 5), data=0xA0000)
    q1 = _t4((1, 2, 1, 8))
    assert lib.bdh_tril_decode(ctypes.byref(q1), ctypes.byref(kp), ctypes.byref(vp), ctypes.byref(o1), None, 0, None) == 1


def test_binding_refuses_cpu_tensors_loudly():
    import bdh_hip_ext as ext

    q = torch.zeros(1, 1, 4, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ext.tril_score_v(q, q, q[..., :2])


# ------------------------------------------------------------ dispatch surface
@pytest.fixture
def K(monkeypatch):
    import kernels

    for var in ("BDH_ATTN_IMPL", "BDH_ATTN_AUTO", "BDH_ATTN_AUTO_THRESHOLD", "BDH_ATTN_AUTO_COLD_THRESHOLD",
                "BDH_ATTN_AUTOGRAD", "BDH_ROPE_IMPL"):
        monkeypatch.delenv(var, raising=False)
    return kernels


def test_impl_resolution_contract(K, monkeypatch):
    assert K.resolve_attn_impl() == "eager"
    assert K.resolve_attn_impl("HIP ") == "hip"
    for bad in ("triton", "blocked", "cuda", "fused"):
        with pytest.raises(ValueError, match="BDH_ATTN_IMPL must be eager|hip"):
            K.resolve_attn_impl(bad)
    monkeypatch.setenv("BDH_ATTN_IMPL", "hip")
    assert K.resolve_attn_impl() == "hip"
    monkeypatch.setenv("BDH_ATTN_IMPL", "nope")
    with pytest.raises(ValueError):
        K.resolve_attn_impl()
    assert K.resolve_rope_impl("hip") == "hip"
    with pytest.raises(ValueError, match="BDH_ROPE_IMPL"):
        K.resolve_rope_impl("fused")


def test_auto_thresholds_contract(K, monkeypatch):
    assert K.attn_auto_threshold() == 512 and K.attn_auto_cold_threshold() == 512
    monkeypatch.setenv("BDH_ATTN_AUTO_THRESHOLD", "100")
    assert K.attn_auto_cold_threshold() == 100
    monkeypatch.setenv("BDH_ATTN_AUTO_COLD_THRESHOLD", "7")
    assert K.attn_auto_cold_threshold() == 7
    monkeypatch.setenv("BDH_ATTN_AUTO_THRESHOLD", "-1")
    with pytest.raises(ValueError, match=">= 0"):
        K.attn_auto_threshold()
    monkeypatch.setenv("BDH_ATTN_AUTO_THRESHOLD", "abc")
    with pytest.raises(ValueError, match="int"):
        K.attn_auto_threshold()
    monkeypatch.setenv("BDH_ATTN_AUTO_THRESHOLD", "512")
    monkeypatch.setenv("BDH_ATTN_AUTO", "1")
    # strict '>' gate; without a GPU the long path stays eager (never a silent CPU 'hip')
    assert K.resolve_cold_impl(7) == "eager"
    assert K.resolve_decode_impl(513) == ("hip" if torch.cuda.is_available() else "eager")


def test_auto_keeps_eager_for_operands_hip_cannot_take(K, monkeypatch):
    """AUTO never switches to a backend that would raise: with the library and a
    device reported present, CPU tensors (or float64) above the threshold still
    take the eager path and return its result (reference AUTO falls back to a
    working path, attention_dispatch.py:203-260)."""
    from kernels import attention_dispatch as d, hip_attn

    monkeypatch.setattr(hip_attn, "hip_available", lambda: True)
    monkeypatch.setenv("BDH_ATTN_AUTO", "1")
    monkeypatch.setenv("BDH_ATTN_AUTO_THRESHOLD", "4")
    g = torch.Generator().manual_seed(0)
    q = torch.relu(0.32 * torch.randn(1, 2, 9, 8, generator=g))
    v = torch.randn(1, 1, 9, 5, generator=g)
    assert d.resolve_cold_impl(9, tensors=(q, q, v)) == "eager"
    assert d.resolve_cold_impl(9) == "hip"  # no operands given: library and device decide
    assert d.resolve_decode_impl(9, tensors=(q[:, :, :1], q, v)) == "eager"
    want = K.bdh_attn(q, q, v, impl="eager")
    assert torch.equal(K.bdh_attn(q, q, v), want)
    assert torch.equal(K.bdh_attn_decode(q[:, :, -1:], q, v), K.bdh_attn_decode(q[:, :, -1:], q, v, impl="eager"))
    assert torch.equal(K.bdh_attn_past(q[:, :, 4:], q, v, 4), K.bdh_attn_past(q[:, :, 4:], q, v, 4, impl="eager"))
    f = K.get_freqs(8)
    assert torch.equal(K.bdh_attn_rope(q, v, f, 0), K.bdh_attn_rope(q, v, f, 0, impl="eager"))
    q64 = q.double()
    assert d.resolve_cold_impl(9, tensors=(q64, q64, v.double())) == "eager"
    # an explicit hip is never replaced
    with pytest.raises(RuntimeError):
        K.bdh_attn(q, q, v, impl="hip")


def test_native_module_name_of_the_reference_dispatches_by_device():
    """``bdh_cuda_ext`` (the import name of reference kernels/cuda_attn.py:84-88)
    reports has_cuda and runs CPU tensors through its torch CPU entries, which
    reproduce the reference's known answers exactly and accumulate 16-bit inputs
    in fp32 (tril_attn_bind.cpp:29,32)."""
    import bdh_cuda_ext as ce
    import bdh_hip_ext as ext

    assert ce.has_cuda is True and ce.has_hip is True and ce.lib_path == ext.lib_path
    ka = json.loads((GOLDEN / "known_answers.json").read_text())
    c = ka["raw_tril_fwd_bwd"]
    q, k, v = (torch.tensor(c[n]) for n in ("q", "k", "v"))
    assert torch.equal(ce.tril_score_v(q, k, v), torch.tensor(c["out"]))
    assert torch.equal(ext.tril_score_v_cpu(q, k, v), torch.tensor(c["out"]))
    d = ka["decode_raw"]
    qd, kd, vd = (torch.tensor(d[n]) for n in ("q", "k_past", "v_past"))
    assert torch.equal(ce.tril_decode(qd, kd, vd), torch.tensor(d["out"]))
    g = torch.Generator().manual_seed(3)
    x = torch.relu(0.32 * torch.randn(2, 2, 40, 32, generator=g))
    vv = torch.randn(2, 1, 40, 16, generator=g)
    want = O.tril_score_v_cpu(O.bf16_round(x.numpy()), O.bf16_round(x.numpy()), O.bf16_round(vv.numpy()))
    got = ce.tril_score_v(x.bfloat16(), x.bfloat16(), vv.bfloat16())
    assert got.dtype == torch.bfloat16
    # fp32 accumulation: only the final rounding to bf16 separates it from the fp32 oracle
    assert float(np.abs(got.float().numpy() - want).max() / np.abs(want).max()) < 2 ** -8
    with pytest.raises(RuntimeError, match="CPU"):
        ext.tril_score_v_cpu(x.to("meta"), x.to("meta"), vv.to("meta"))


def test_eager_paths_match_oracle_and_known_answers(K):
    ka = json.loads((GOLDEN / "known_answers.json").read_text())
    c = ka["raw_tril_fwd_bwd"]
    Q = torch.tensor(c["q"], requires_grad=True)
    Kt = torch.tensor(c["k"], requires_grad=True)
    V = torch.tensor(c["v"], requires_grad=True)
    out = K.strict_tril_attn(Q, Kt, V, impl="eager", use_fn=True)
    assert torch.equal(out, torch.tensor(c["out"]))
    out.sum().backward()
    assert torch.equal(Q.grad, torch.tensor(c["dq"]))
    assert torch.equal(Kt.grad, torch.tensor(c["dk"]))
    assert torch.equal(V.grad, torch.tensor(c["dv"]))
    c = ka["self_attn_single_query"]
    Q = torch.tensor(c["q"], requires_grad=True)
    V = torch.tensor(c["v"], requires_grad=True)
    out = K.strict_tril_attn(Q, Q, V, impl="eager", use_fn=True)
    out.backward(torch.tensor(c["dout"]))
    assert torch.equal(Q.grad, torch.tensor(c["dq_merged"]))
    assert torch.equal(V.grad, torch.tensor(c["dv"]))
    d = ka["decode_raw"]
    assert torch.equal(K.bdh_attn_decode(torch.tensor(d["q"]), torch.tensor(d["k_past"]), torch.tensor(d["v_past"])),
                       torch.tensor(d["out"]))


def test_hip_on_cpu_tensors_raises_runtime_error(K):
    q = torch.randn(1, 2, 5, 4)
    v = torch.randn(1, 1, 5, 3)
    with pytest.raises(RuntimeError):
        K.bdh_attn(q, q, v, impl="hip")
    with pytest.raises(RuntimeError):
        K.bdh_attn_decode(q[:, :, :1], q, v, impl="hip")
    with pytest.raises(RuntimeError):
        K.bdh_rope_rotate(q, *K.rope_cos_sin(5, 0, K.get_freqs(4)), impl="hip")
    with pytest.raises(ValueError, match="heads"):  # shape contract checked before the device check
        K.bdh_attn(q, q, torch.randn(1, 3, 5, 3), impl="hip")


def test_rope_validation_contract(K):
    v = torch.randn(1, 1, 3, 6)
    c, s = K.rope_cos_sin(3, 0, K.get_freqs(6))
    with pytest.raises(ValueError, match="even"):
        K.bdh_rope_rotate(torch.randn(1, 1, 3, 5), c[..., :5], s[..., :5])
    with pytest.raises(ValueError, match="last dim"):
        K.bdh_rope_rotate(v, c[..., :4], s[..., :4])
    with pytest.raises(ValueError, match="alias"):
        K.bdh_rope_rotate(v, c, s, out=v)
    with pytest.raises(ValueError, match="shape/device"):
        K.bdh_rope_rotate(v, c, s, out=torch.empty(1, 1, 3, 4))
    cp, sp = c.reshape(1, 1, 3, 3, 2), s.reshape(1, 1, 3, 3, 2)
    with pytest.raises(ValueError, match="trailing dims"):
        K.bdh_rope_rotate_paired(v, cp[..., :2, :], sp[..., :2, :])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_eager_rope_matches_oracle_bit_exactly(K, dtype):
    N, T, start = 32, 9, 5
    f = K.get_freqs(N)
    assert np.array_equal(f.numpy(), O.get_freqs(N)) or np.allclose(f.numpy(), O.get_freqs(N), rtol=2e-7)
    x = torch.randn(2, 3, T, N).to(dtype)
    c, s = K.rope_cos_sin(T, start, f)
    got = K.bdh_rope_rotate(x, c, s).float().numpy()
    want = O.rope_rotate(x.float().numpy(), c.numpy(), s.numpy(), bf16=(dtype == torch.bfloat16))
    assert np.array_equal(got, want)
    # phases: torch (reference formula) and oracle give the same cos/sin bits
    oc, os_ = O.rope_cos_sin(T, start, f.numpy())
    assert np.allclose(c[0, 0].numpy(), oc, atol=1e-6) and np.allclose(s[0, 0].numpy(), os_, atol=1e-6)


def test_bdh_attn_rope_eager_matches_oracle(K):
    g = torch.Generator().manual_seed(0)
    x = torch.relu(0.32 * torch.randn(2, 2, 30, 16, generator=g))
    v = torch.randn(2, 1, 30, 8, generator=g)
    f = K.get_freqs(16)
    got = K.bdh_attn_rope(x, v, f, 2).numpy()
    want, _ = O.tril_rope_score_v(x.numpy(), v.numpy(), f.numpy(), 2)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


# -------------------------------------------------------------- fixtures
def test_golden_fixtures_reproduce():
    z = np.load(GOLDEN / "fixtures.npz")  # allow_pickle defaults to False
    x, k, v, dy, f, start = z["x"], z["k"], z["v"], z["dy"], z["freqs"], int(z["rope_start"])
    tol = dict(rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(O.tril_score_v_cpu(x, k, v), z["cold_out"], **tol)
    out, qr = O.tril_rope_score_v(x, v, f, start)
    np.testing.assert_allclose(out, z["rope_out"], **tol)
    np.testing.assert_allclose(qr, z["qr"], **tol)
    dx, dv = O.tril_rope_score_v_backward(x, v, dy, f, start)
    np.testing.assert_allclose(dx, z["rope_dx"], **tol)
    np.testing.assert_allclose(dv, z["rope_dv"], **tol)
    S = int(z["dec_S"])
    np.testing.assert_allclose(O.tril_decode_cpu(z["dec_q"], z["qr"][:, :, :S], v[:, :, :S]), z["dec_out"], **tol)
    assert np.array_equal(O.rope_rotate(z["x_bf16"], z["cos"], z["sin"], bf16=True), z["rope_bf16"])


# --------------------------------------------------------- entry points
def test_bench_refuses_multi_gpu():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr


def test_graft_entry_has_build_and_smoke():
    sys.path.insert(0, str(ROOT))
    import __graft_entry__ as g

    assert callable(g.build) and callable(g.smoke)
