"""Config 5 at its real shapes and settings: the synthetic 12-layer d=2048
parameter set and per-step gradients of bench.py (same seeds), the Muon arm
and the Shampoo arm teacher-forced against the numpy oracle at steps 0, 1,
20 and 39 of the 40-step run (two root refreshes, a stale-root step
between them and the last step, 19 steps after the second refresh).

A subset of the matrices is optimised (every matrix's update is independent
of the others'), chosen so that the harnesses run the same stacked
launches as on the full set, and the CPU oracle stays within seconds:
  Muon arm     the eight attention matrices of layers 0 and 1 [2048, 2048]
               (one stacked fp32 NS5 of 8, as the bench's 48), l0.up, l1.up
               [8192, 2048] and l0.down, l1.down [2048, 8192] (stacks of 2),
               and the tied embedding [32000, 2048] on AdamW;
  Shampoo arm  the four attention matrices of layer 3 [2048, 2048] (factor
               updates stacked 4 per side, the refresh's 8 roots in one
               inverse_matrix_root_each call) with the reference's defaults
               that config 5 keeps: beta2 0.999, eps 1e-8, root_method
               "auto", root_dtype float64, plus precondition_frequency 20,
               graft "adagrad", max_preconditioner_dim 4096.
Which stacks ran is checked from the ops calls and, for the NS5 and factor
kernels, from the library's launch counts.
The oracle's Shampoo roots are float64 eigh, the reference's "auto"
(pytorch_opt/ops/reference.py:64-67); the GPU's "auto" runs the float64
coupled Newton kernels, so the roots are compared by the residual
‖X⁴(A + εI) − I‖_F/√n (within 1e-3 of the oracle's) and elementwise.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
CHECK = (0, 1, 20, 39)
STEPS = 40


def _params_and_grads():
    import bench

    P = bench.config5_params(torch, torch.device(DEV))
    return P, lambda step: bench.set_grads(torch, P, step, torch.device(DEV))


def _np(t):
    return t.detach().float().cpu().numpy() if t.dtype != torch.float64 else t.detach().cpu().numpy()


def _residual(X, A, eps):
    n = A.shape[-1]
    M = A.double() + eps * torch.eye(n, dtype=torch.float64, device=A.device)
    Xd = X.double()
    X2 = Xd @ Xd
    return float(((X2 @ X2) @ M - torch.eye(n, dtype=torch.float64, device=A.device)).norm() / n ** 0.5)


def _record_calls(monkeypatch, name, describe):
    """Wrap pytorch_opt.ops.<name>, appending describe(args) per call."""
    from pytorch_opt import ops

    seen = []
    real = getattr(ops, name)

    def wrapper(*args, **kwargs):
        seen.append(describe(*args))
        return real(*args, **kwargs)

    monkeypatch.setattr(ops, name, wrapper)
    return seen


def test_config5_muon_arm_teacher_forced(native_backend, monkeypatch):
    from oracle import optim_oracle as oopt
    from pytorch_opt import Muon

    P, set_grads = _params_and_grads()
    mats = [f"l{l}.{k}" for l in (0, 1) for k in ("q", "k", "v", "o")] + ["l0.up", "l1.up", "l0.down", "l1.down"]
    opt = Muon([{"params": [P[n] for n in mats]}, {"params": [P["emb"]], "use_muon": False}], lr=0.02)
    g_adam = opt.param_groups[1]
    ns_calls = _record_calls(monkeypatch, "newton_schulz_orthogonalize", lambda G, *a: tuple(G.shape))
    for step in range(STEPS):
        set_grads(step)
        if step not in CHECK:
            opt.step()
            continue
        if step == CHECK[-1]:  # launches of one step: 3 stacks x 5 iterations per NS5 kernel
            native_backend.prof_reset()
            native_backend.prof_enable(True)
        want = {}
        for n in mats:
            p = P[n]
            st = opt.state[p]
            buf = _np(st["momentum_buffer"]) if "momentum_buffer" in st else np.zeros(p.shape, np.float32)
            want[n] = oopt.muon_matrix_step(_np(p), _np(p.grad), buf, lr=0.02)
        e = P["emb"]
        st = opt.state[e]
        m = _np(st["exp_avg"]) if "exp_avg" in st else np.zeros(e.shape, np.float32)
        v = _np(st["exp_avg_sq"]) if "exp_avg_sq" in st else np.zeros(e.shape, np.float32)
        lr = g_adam["lr"] if g_adam.get("use_preconditioner") is False else g_adam["adamw_lr"]
        wd = g_adam["weight_decay"] if g_adam.get("use_preconditioner") is False else g_adam["adamw_wd"]
        want_e = oopt.adamw_step(_np(e), _np(e.grad), m, v, st.get("step", 0) + 1, lr, g_adam["adamw_betas"],
                                 g_adam["adamw_eps"], wd)
        del ns_calls[:]
        opt.step()
        assert sorted(ns_calls) == [(2, 2048, 8192), (2, 8192, 2048), (8, 2048, 2048)], (step, ns_calls)
        if step == CHECK[-1]:
            torch.cuda.synchronize()
            native_backend.prof_enable(False)
            for kind in ("ns5_gram", "ns5_square", "ns5_update"):
                assert native_backend.prof_query(kind)[1] == 15, kind
        for n in mats:
            p_w, buf_w, _ = want[n]
            np.testing.assert_allclose(_np(opt.state[P[n]]["momentum_buffer"]), buf_w, atol=1e-7, err_msg=n)
            err = np.abs(_np(P[n]) - p_w).max()
            assert err < 1e-5, (step, n, err)
        assert np.abs(_np(e) - want_e[0]).max() < 1e-6, step
        np.testing.assert_allclose(_np(opt.state[e]["exp_avg_sq"]), want_e[2], rtol=1e-5, atol=1e-12)


def test_config5_shampoo_arm_teacher_forced(native_backend, monkeypatch):
    """Each stage of a step starts from the GPU's result of the stage before
    (per-stage teacher forcing): at ε = 1e-8 the float32 rounding of a
    2048² factor G·Gᵀ (spectral norm ~1e-8) is as large as its smallest
    eigenvalues plus ε, so roots of two independently rounded factors
    differ in those directions whatever computes them; the roots are
    therefore checked from the GPU's own factors."""
    from oracle import ops_oracle as oo
    from oracle import optim_oracle as oopt
    from pytorch_opt import Shampoo

    P, set_grads = _params_and_grads()
    mats = [f"l3.{k}" for k in ("q", "k", "v", "o")]
    kw = dict(lr=0.03, beta2=0.999, eps=1e-8, precondition_frequency=20, graft="adagrad")
    opt = Shampoo([{"params": [P[n] for n in mats]}], max_preconditioner_dim=4096, **kw)
    assert opt.param_groups[0]["root_method"] == "auto" and opt.param_groups[0]["root_dtype"] == torch.float64
    root_calls = _record_calls(monkeypatch, "inverse_matrix_root_each", lambda A, *a: tuple(A.shape))
    kron_calls = _record_calls(monkeypatch, "kron_factor_update_batched_", lambda Ls, Rs, Gs, *a: len(Gs))
    for step in range(STEPS):
        set_grads(step)
        if step not in CHECK:
            opt.step()
            continue
        del root_calls[:], kron_calls[:]
        native_backend.prof_reset()
        native_backend.prof_enable(True)
        before = {}
        for n in mats:
            st = opt.state[P[n]]
            z = np.zeros(P[n].shape, np.float32)
            before[n] = {k: (_np(st[k]) if k in st else z) for k in ("L", "R", "graft_acc")}
            before[n].update(p=_np(P[n]), g=_np(P[n].grad), fu=st.get("factor_updates", 0),
                             L_root=_np(st["L_root"]) if "L_root" in st else None,
                             R_root=_np(st["R_root"]) if "R_root" in st else None)
        opt.step()
        torch.cuda.synchronize()
        native_backend.prof_enable(False)
        assert kron_calls == [4], (step, kron_calls)
        assert native_backend.prof_query("kron_left")[1] == 1 and native_backend.prof_query("kron_right")[1] == 1
        assert root_calls == ([(8, 2048, 2048)] if step % 20 == 0 else []), (step, root_calls)
        for n in mats:
            st, b = opt.state[P[n]], before[n]
            # 1. factor update from the previous factors
            L_w, R_w = oo.kron_factor_update(b["L"], b["R"], b["g"], 0.999)
            np.testing.assert_allclose(_np(st["L"]), L_w, rtol=1e-5, atol=1e-9, err_msg=n)
            np.testing.assert_allclose(_np(st["R"]), R_w, rtol=1e-5, atol=1e-9, err_msg=n)
            refresh = step % 20 == 0
            if refresh:
                # 2. roots of the GPU's factors: float64 eigh (the reference's
                #    auto) against the GPU's float64 coupled Newton
                bc = 1.0 - 0.999 ** st["factor_updates"]
                for side in ("L", "R"):
                    A = st[side] / bc
                    want_root, _ = oo.inverse_root(_np(A), 4, damping=1e-8, method="eigh", root_dtype=np.float64)
                    got_root = st[side + "_root"]
                    r_g = _residual(got_root, A, 1e-8)
                    r_o = _residual(torch.from_numpy(want_root).to(DEV), A, 1e-8)
                    rel = np.linalg.norm(_np(got_root) - want_root) / np.linalg.norm(want_root)
                    print(f"step {step} {n} {side}: residual hip {r_g:.4e} oracle {r_o:.4e}, rel diff {rel:.2e}")
                    assert abs(r_g - r_o) <= 1e-3, (step, n, side, r_g, r_o)
                    assert rel < 1e-6, (step, n, side, rel)
            # 3. apply, AdaGrad graft and update from the GPU's factors and roots
            roots = (_np(st["L_root"]), _np(st["R_root"])) if refresh else None
            p_w = oopt.shampoo_matrix_step(b["p"], b["g"], b["L"], b["R"], b["L_root"], b["R_root"],
                                           b["graft_acc"], step, b["fu"], root_method="eigh",
                                           factors=(_np(st["L"]), _np(st["R"])), roots=roots, **kw)[0]
            err = np.abs(_np(P[n]) - p_w).max()
            assert err < 1e-5, (step, n, err)
