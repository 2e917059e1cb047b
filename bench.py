"""Benchmark of the pytorch_opt.ops hot path on one MI355X.

Headline workload (one "step"): NS5, 5 quintic iterations, on 32 bf16
matrices 4096x4096 plus 32 bf16 matrices 4096x11008 (Llama-7B-like
projection shapes); inputs are the Nesterov momentum (β=0.95) of three
seeded N(0, 1e-3) gradients, resident in HBM before timing. Two batched calls
of pytorch_opt.ops.newton_schulz_orthogonalize through the HIP library.

The JSON line carries the headline (algorithmic TFLOP/s, LAWN-41 counting,
timed with no instrumentation), the roofline of the dominant kernel (a
second pass with HIP events recorded on each launch's stream inside the
library), the reference's CPU path (pytorch_opt.ops.reference, the ATen op
sequence of the reference's ops, on CPU tensors) on a bounded sample of
the same workload, and secondary figures:
  single_4096   one 4096x4096 NS5;
  factors       Kronecker EMA update of fp32 G 4096² and the K-FAC Gram
                AᵀA/n of bf16 A 16384x4096 into fp32;
  roots         inverse 4th roots (coupled Newton, fp32) of SPD n = 1024 /
                2048 / 4096 with λ log-uniform in [1e-6, 1], ε = 1e-6;
  optimizer     Muon + Shampoo steps on the synthetic 12-layer d=2048
                parameter set (40 steps each), SOAP on its 48 attention
                matrices (one refresh period, 10 steps; and with
                basis_refresh="power", whose refreshes after the first are
                one subspace-iteration step, timed at step 20), with the
                CPU path's per-step estimate from a bounded sample;
  kfac          K-FAC and EKFAC steps on 4 x Linear(2048, 2048), 8192
                tokens (one inv_every = 10 period), with a CPU estimate.
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "pytorch-opt_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK = {"bf16": 2516.6, "fp32": 157.3, "fp64": 78.6}  # MI355X dense MFMA TFLOP/s
SHAPES = [(32, 4096, 4096, 1000), (32, 4096, 11008, 2000)]  # (batch, rows, cols, seed base)


def ns5_flops(m, n, steps=5):
    m, n = min(m, n), max(m, n)
    return steps * (m * (m + 1) * n + m * m * (m + 1) + 2 * m * m * n)


def ns5_kernel_flops(kind, m, n):
    """Algorithmic flops of one NS5 iteration's launch of `kind`, per matrix."""
    m, n = min(m, n), max(m, n)
    return {"ns5_gram": m * (m + 1) * n, "ns5_square": m * m * (m + 1), "ns5_update": 2 * m * m * n}[kind]


def soap_matrix_flops(m, n):
    """Algorithmic flops of one SOAP step (no refresh) of an m x n matrix: the
    factor update (two symmetric products) and three two-sided rotations."""
    return m * (m + 1) * n + n * (n + 1) * m + 3 * (2 * m * m * n + 2 * m * n * n)


def cpu_setup(torch):
    """Threads for the CPU baseline: the physical cores, capped by the
    host's CPU share for this job (OMP_NUM_THREADS when set). Returns the
    facts the report states."""
    try:
        import psutil

        physical = psutil.cpu_count(logical=False) or os.cpu_count() or 1
    except ImportError:
        physical = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(physical, share) if share > 0 else physical
    torch.set_num_threads(threads)
    return {"threads": torch.get_num_threads(), "physical_cores": physical, "nproc": os.cpu_count(),
            "model": cpu_model()}


def cpu_model():
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        return next((l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("Model name")), "")
    except Exception:
        return ""


def timed(fn, reps=1):
    """Seconds per call: one warm-up call, then the median of `reps` calls."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def warm_gpu(torch, fn, min_s=0.06):
    """Run fn back to back for at least min_s seconds. After any pause the
    device clocks take ~20-30 ms of work to leave their idle state (one 4096²
    NS5 measured 1.21-1.32 ms in its first 20 calls, then 1.175-1.18 ms
    sustained over the next second), so short timings start from here."""
    t0 = time.perf_counter()
    while True:
        fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= min_s:
            return


def gpu_ms_per_call(torch, fn, min_s=0.05, min_reps=5):
    """Milliseconds per call of fn on the current stream, after warm_gpu:
    enough back-to-back calls to fill about min_s seconds, timed by events."""
    warm_gpu(torch, fn)
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    reps = max(min_reps, int(min_s / max(time.perf_counter() - t0, 1e-6)))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


# ------------------------------------------------------------ headline (config 2)

def make_ns5_inputs(torch, batch, rows, cols, seed0, dev):
    out = torch.empty(batch, rows, cols, dtype=torch.bfloat16, device=dev)
    for i in range(batch):
        g = torch.Generator(device=dev).manual_seed(seed0 + i)
        buf = torch.zeros(rows, cols, device=dev)
        gt = None
        for _ in range(3):
            gt = 1e-3 * torch.randn(rows, cols, generator=g, device=dev)
            buf.mul_(0.95).add_(gt)
        out[i] = (gt + 0.95 * buf).bfloat16()
    return out


def cpu_baseline_ns5(torch, inputs, host):
    """The reference's CPU path for NS5: pytorch_opt.ops.reference (the same
    ATen op sequence as the reference's ops, fp32 work on the bf16 input) on
    CPU tensors, one matrix of each shape, time scaled x32 each."""
    from pytorch_opt.ops import reference as ref

    total_s = 0.0
    for (batch, _, _, _), G in zip(SHAPES, inputs):
        x = G[0].cpu()
        total_s += timed(lambda: ref.newton_schulz_orthogonalize(x)) * batch
    flops = sum(b * ns5_flops(r, c) for b, r, c, _ in SHAPES)
    return {"value": round(flops / total_s / 1e12, 4), "unit": "TFLOP/s", "cores": host["threads"], "kind": "port",
            "sample": "pytorch_opt.ops.reference NS5 (torch/ATen on CPU tensors, fp32) on 1 matrix 4096x4096 + 1 "
                      f"matrix 4096x11008 of the same inputs, time x32 each: est. {total_s:.1f} s for the full "
                      f"workload; {host['threads']} threads (torch.get_num_threads), {host['physical_cores']} "
                      f"physical cores, nproc {host['nproc']}, {host['model']}"}


# ------------------------------------------------------------ config 3 / 4

def bench_factors(torch, ops, hip, dev, cpu):
    """Kronecker EMA update (fp32 G 4096², β 0.95) and K-FAC Gram (bf16 A 16384x4096)."""
    import numpy as np

    g = torch.Generator(device=dev).manual_seed(2)
    G0 = 1e-2 * torch.randn(4096, 4096, generator=g, device=dev)
    G = 1e-2 * torch.randn(4096, 4096, generator=g, device=dev)
    L, R = G0 @ G0.T, G0.T @ G0
    g3 = torch.Generator(device=dev).manual_seed(3)
    A = torch.randn(16384, 4096, generator=g3, device=dev).bfloat16()
    F = torch.zeros(4096, 4096, device=dev)
    res = {}
    for name, fn, flops, peak, kinds in [
        ("kron_update_fp32_4096", lambda: ops.kron_factor_update_(L, R, G, beta2=0.95), 2 * 4096 * 4097 * 4096,
         "fp32", ("kron_left", "kron_right")),
        ("kfac_gram_bf16_16384x4096", lambda: ops.gram_update_(F, A, beta=0.95, alpha=0.05 / 16384),
         4096 * 4097 * 16384, "bf16", ("gram_update", "gram_update_direct"))]:
        wall = gpu_ms_per_call(torch, fn) / 1e3  # uninstrumented
        hip.prof_reset()
        hip.prof_enable(True)
        reps = 10
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        hip.prof_enable(False)
        kms = sum(hip.prof_query(k)[0] for k in kinds) / reps
        res[name] = {"ms": round(wall * 1e3, 3), "kernel_ms": round(kms, 3),
                     "tflops": round(flops / wall / 1e12, 2),
                     "pct_peak": round(100 * flops / wall / 1e12 / PEAK[peak], 2), "peak_dtype": peak}
    if cpu:
        from pytorch_opt.ops import reference as ref

        Gc, Lc, Rc = G.cpu(), L.cpu(), R.cpu()
        t = timed(lambda: ref.kron_factor_update_(Lc.clone(), Rc.clone(), Gc, beta2=0.95), reps=3)
        res["kron_update_fp32_4096"]["cpu_ms"] = round(t * 1e3, 1)
        Ac, Fc = A[:4096].cpu(), F.cpu()  # a quarter of the tokens, scaled x4
        t = timed(lambda: ref.gram_update_(Fc, Ac, beta=0.95, alpha=0.05 / 16384), reps=3) * 4
        res["kfac_gram_bf16_16384x4096"]["cpu_ms"] = round(t * 1e3, 1)
        res["cpu_note"] = ("pytorch_opt.ops.reference on CPU tensors (fp32 ATen, median of 3); the Gram times "
                           "4096 of the 16384 rows and scales x4")
    return res


def bench_roots(torch, hip, dev, cpu):
    """Coupled-Newton inverse 4th roots, fp32, n = 1024 / 2048 / 4096, with
    the numpy oracle's residual and iteration count on the same inputs."""
    res = {}
    try:
        with open(os.path.join(ROOT, "tests", "golden", "root_config4.json")) as f:
            golden_roots = json.load(f)["cases"]
    except (OSError, ValueError, KeyError):
        golden_roots = {}
    for n in (1024, 2048, 4096):
        g = torch.Generator().manual_seed(4)
        Q, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
        g5 = torch.Generator().manual_seed(5)
        lam = 10 ** (-6 * torch.rand(n, generator=g5, dtype=torch.float64))
        A = ((Q * lam) @ Q.T).float().to(dev)
        warm_gpu(torch, lambda: hip.inverse_matrix_root_iters(A, 4, 1e-6, "newton", False, 100, 1e-10))
        t0 = time.perf_counter()
        X, iters = hip.inverse_matrix_root_iters(A, 4, 1e-6, "newton", False, 100, 1e-10)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        Xd = X.double()
        X2 = Xd @ Xd
        M = A.double() + 1e-6 * torch.eye(n, dtype=torch.float64, device=dev)
        resid = float(((X2 @ X2) @ M - torch.eye(n, dtype=torch.float64, device=dev)).norm() / n ** 0.5)
        # LAWN-41 count per iteration, as the kernels compute it: X·Mi, Mi², Mi⁴ and
        # Mi⁴·Mk are all products of commuting polynomials in M, so each is a
        # symmetric product on upper tiles, n²(n+1) flops
        it_flops = 4 * n * n * (n + 1)
        tflops = iters * it_flops / wall / 1e12
        entry = {"ms": round(wall * 1e3, 2), "iterations": iters, "ms_per_iter": round(wall * 1e3 / max(iters, 1), 3),
                 "residual": float(f"{resid:.4e}"), "alg_flops_per_iter": it_flops,
                 "tflops": round(tflops, 2), "frac_fp32_peak": round(tflops / PEAK["fp32"], 4)}
        gold = golden_roots.get(str(n))
        if gold is not None:  # the numpy oracle's float32 run, tests/golden/root_config4.json
            entry["oracle_residual"] = float(f"{gold['residual']:.4e}")
            entry["oracle_iterations"] = gold["iterations"]
        if cpu and n == 1024:
            from pytorch_opt.ops import reference as ref

            Ac = A.cpu()
            t = timed(lambda: ref.inverse_matrix_root(Ac, 4, 1e-6, "newton", torch.float32, 100, 1e-10))
            entry["cpu_ms"] = round(t * 1e3, 1)
        res[f"n{n}"] = entry
    return res


# ------------------------------------------------------------ config 5

def config5_shapes():
    mats, vecs = [], []
    for l in range(12):
        for nm in ("q", "k", "v", "o"):
            mats.append((f"l{l}.{nm}", (2048, 2048), "attn"))
        mats.append((f"l{l}.up", (8192, 2048), "mlp"))
        mats.append((f"l{l}.down", (2048, 8192), "mlp"))
        for nm in ("ln1.w", "ln1.b", "ln2.w", "ln2.b"):
            vecs.append((f"l{l}.{nm}", (2048,)))
    vecs += [("lnf.w", (2048,)), ("lnf.b", (2048,))]
    return mats, vecs


def config5_params(torch, dev):
    mats, vecs = config5_shapes()
    g = torch.Generator(device=dev).manual_seed(6)
    P = {}
    for name, shape, _ in mats:
        P[name] = torch.nn.Parameter(0.02 * torch.randn(shape, generator=g, device=dev))
    for name, shape in vecs:
        P[name] = torch.nn.Parameter(torch.ones(shape, device=dev) if name.endswith(".w")
                                     else torch.zeros(shape, device=dev))
    P["emb"] = torch.nn.Parameter(0.02 * torch.randn(32000, 2048, generator=g, device=dev))
    return P


def set_grads(torch, P, step, dev):
    g = torch.Generator(device=dev).manual_seed(10_000 + step)
    for p in P.values():
        p.grad = 1e-3 * torch.randn(p.shape, generator=g, device=dev)


def bench_optimizer(torch, ops, hip, dev, steps, cpu):
    from pytorch_opt import SOAP, Muon, Shampoo

    mats, vecs = config5_shapes()
    kind = {n: k for n, _, k in mats}
    out = {}

    def run(make_opt, n_steps=steps):
        P = config5_params(torch, dev)
        opt = make_opt(P)
        total, per = 0.0, []
        for t in range(n_steps):
            set_grads(torch, P, t, dev)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            opt.step()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            per.append(dt)
            total += dt
        del P, opt
        torch.cuda.empty_cache()
        return total / n_steps, per

    def make_muon(P):
        routed = [P[n] for n, _, _ in mats]
        rest = [P[n] for n, _ in vecs] + [P["emb"]]
        return Muon([{"params": routed}, {"params": rest, "use_muon": False}], lr=0.02)

    def make_shampoo(P):
        attn = [P[n] for n, _, _ in mats if kind[n] == "attn"]
        rest = [P[n] for n, _, _ in mats if kind[n] == "mlp"] + [P[n] for n, _ in vecs] + [P["emb"]]
        return Shampoo([{"params": attn}, {"params": rest, "use_preconditioner": False, "lr": 3e-4}],
                       max_preconditioner_dim=4096, precondition_frequency=20, graft="adagrad")

    def make_soap(P, basis_refresh="eigh"):
        attn = [P[n] for n, _, _ in mats if kind[n] == "attn"]
        rest = [P[n] for n, _, _ in mats if kind[n] == "mlp"] + [P[n] for n, _ in vecs] + [P["emb"]]
        return SOAP([{"params": attn}, {"params": rest, "use_preconditioner": False}], lr=3e-3,
                    max_preconditioner_dim=4096, precondition_frequency=10, basis_refresh=basis_refresh)

    m_mean, _ = run(make_muon)
    s_mean, s_per = run(make_shampoo)
    # SOAP: one refresh (step 0, 96 fp64 eigh on torch) and 9 plain steps,
    # i.e. one precondition_frequency period
    _, soap_per = run(make_soap, 10)
    out["soap_refresh_step_ms"] = round(soap_per[0] * 1e3, 1)
    out["soap_plain_step_ms"] = round(1e3 * sum(soap_per[1:]) / 9, 2)
    out["soap_step_ms"] = round(1e3 * sum(soap_per) / 10, 2)
    out["soap_plain_alg_tflops"] = round(48 * soap_matrix_flops(2048, 2048) / (sum(soap_per[1:]) / 9) / 1e12, 2)
    # SOAP(basis_refresh="power"): eigh at step 0, then every refresh is
    # one subspace-iteration step per factor (F·Q, shifted CholeskyQR3 in
    # float64); timed at its second such refresh, step 20 (the first pays
    # the process's one-time setup of torch's batched GEMM and
    # factorisations), over the period steps 11..20
    _, pw_per = run(lambda P: make_soap(P, "power"), 21)
    out["soap_power_refresh_step_ms"] = round(pw_per[20] * 1e3, 1)
    out["soap_power_step_ms"] = round(1e3 * sum(pw_per[11:21]) / 10, 2)
    refresh = [s_per[i] for i in range(steps) if i % 20 == 0]
    plain = [s_per[i] for i in range(steps) if i % 20 != 0]
    out["muon_step_ms"] = round(m_mean * 1e3, 2)
    out["shampoo_step_ms"] = round(s_mean * 1e3, 2)
    out["shampoo_refresh_step_ms"] = round(1e3 * sum(refresh) / max(len(refresh), 1), 1)
    out["shampoo_plain_step_ms"] = round(1e3 * sum(plain) / max(len(plain), 1), 2)
    out["muon_plus_shampoo_step_ms"] = round((m_mean + s_mean) * 1e3, 2)
    out["muon_alg_tflops"] = round(sum(ns5_flops(*s) for _, s, _ in mats) / m_mean / 1e12, 2)
    out["steps"] = steps
    if cpu:
        out["cpu"] = cpu_optimizer_estimate(torch, steps, cpu)
        out["speedup_vs_cpu"] = round(out["cpu"]["muon_plus_shampoo_step_ms"] / out["muon_plus_shampoo_step_ms"], 1)
        out["soap_speedup_vs_cpu"] = round(out["cpu"]["soap_step_ms"] / out["soap_step_ms"], 1)
    return out


def cpu_optimizer_estimate(torch, steps, host):
    """Per-step CPU time of the same arms from a bounded sample of the
    reference's CPU path (pytorch_opt.ops.reference ops and torch's AdamW
    update chain on CPU tensors): one NS5 of each shape, one factor update
    + apply, one float64 eigh root (the reference's 'auto'), one rotation,
    one float64 eigh, one AdamW pass over 2048x8192, each scaled by its
    count per step."""
    from pytorch_opt.ops import reference as ref

    g = torch.Generator().manual_seed(0)
    sq = 1e-3 * torch.randn(2048, 2048, generator=g)
    wide = 1e-3 * torch.randn(2048, 8192, generator=g)
    t_ns_sq = timed(lambda: ref.newton_schulz_orthogonalize(sq))
    t_ns_wide = timed(lambda: ref.newton_schulz_orthogonalize(wide))
    L = sq @ sq.T
    t_kron = timed(lambda: ref.kron_factor_update_(L.clone(), L.clone(), sq, beta2=0.999))
    t_apply = timed(lambda: ref.precond_apply_two_sided(L, sq, L))
    t_root = timed(lambda: ref.inverse_matrix_root(L / 0.001, 4, damping=1e-8, method="auto"))
    p, m, v = wide.clone(), torch.zeros_like(wide), torch.zeros_like(wide)
    t_adamw = timed(lambda: ref.adamw_step_(p, wide, m, v, 3e-4, 0.0, (0.9, 0.95), 1e-8, 1))
    per_elem = t_adamw / wide.numel()
    emb_norms = 32000 * 2048 + 12 * 4 * 2048 + 2 * 2048
    mlp = 24 * 2048 * 8192
    muon = 48 * t_ns_sq + 24 * t_ns_wide + per_elem * emb_norms
    plain = 48 * (t_kron + t_apply) + per_elem * (emb_norms + mlp)
    refresh = plain + 96 * t_root
    shampoo = (2 * refresh + (steps - 2) * plain) / steps
    t_rot = timed(lambda: ref.two_sided_product(L, sq, L, transpose_a=True))
    t_eigh = timed(lambda: torch.linalg.eigh(L.double()))
    soap_plain = 48 * (t_kron + 3 * t_rot) + per_elem * (48 * sq.numel() + emb_norms + mlp)
    soap_refresh = soap_plain + 96 * t_eigh + 48 * t_rot
    soap = (soap_refresh + 9 * soap_plain) / 10
    return {"muon_step_ms": round(muon * 1e3, 1), "shampoo_step_ms": round(shampoo * 1e3, 1),
            "muon_plus_shampoo_step_ms": round((muon + shampoo) * 1e3, 1), "soap_step_ms": round(soap * 1e3, 1),
            "soap_plain_step_ms": round(soap_plain * 1e3, 1), "cores": host["threads"], "kind": "port",
            "sample": "pytorch_opt.ops.reference on CPU tensors: 1 NS5 2048², 1 NS5 2048x8192, 1 kron update + "
                      "apply 2048², 1 fp64 eigh root 2048, 1 rotation Q_Lᵀ·G·Q_R 2048², 1 fp64 eigh 2048, AdamW "
                      "over 2048x8192; scaled by per-step counts (48, 24, 48, 96 per refresh, 3x48 rotations, "
                      "elements); Shampoo mean = (2 refresh + (steps-2) plain)/steps, SOAP mean = "
                      f"(refresh + 9 plain)/10; {host['threads']} threads, {host['model']}"}


# ------------------------------------------------------------ K-FAC / EKFAC

KFAC_D, KFAC_DEPTH, KFAC_TOKENS = 2048, 4, 8192


def bench_kfac(torch, dev, cpu):
    """K-FAC (eigh and Newton inverses) and EKFAC optimizer steps on
    4 x Linear(2048, 2048) with bias, 8192 tokens, fp32, over one inv_every =
    10 period after an untimed one: step 0 refreshes the 8 damped inverses /
    eigenbases (float64 eigh of 2049² and 2048², batched, or the batched
    coupled Newton iteration in fp32 with inverse_method="newton"),
    steps 1-9 only precondition (two MFMA products per layer) and update.
    The backward-hook factor statistics are outside opt.step() and are timed
    by the K-FAC Gram line of `factors`."""
    from pytorch_opt import EKFAC, KFAC

    d, depth, tokens = KFAC_D, KFAC_DEPTH, KFAC_TOKENS
    flops = depth * (2 * d * d * (d + 1) + 2 * d * (d + 1) * (d + 1))  # iG·V, (iG·V)·iA per layer
    out = {"workload": f"{depth} x Linear({d}, {d}) + bias, {tokens} tokens, fp32, inv_every 10"}
    arms = (("kfac", KFAC, {}), ("kfac_newton", KFAC, {"inverse_method": "newton"}), ("ekfac", EKFAC, {}))
    for name, cls, kw in arms:
        torch.manual_seed(7)
        model = torch.nn.Sequential(*[torch.nn.Linear(d, d) for _ in range(depth)]).to(dev)
        opt = cls(model, lr=1e-3, damping=1e-3, inv_every=10, **kw)
        X = torch.randn(tokens, d, device=dev)
        per = []
        for _ in range(20):  # one untimed period, then one timed period starting with a refresh
            opt.zero_grad(set_to_none=True)
            (0.5 * model(X).pow(2).sum() / tokens).backward()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            opt.step()
            torch.cuda.synchronize()
            per.append(time.perf_counter() - t0)
        per = per[10:]
        plain = sum(per[1:]) / 9
        out[name] = {"refresh_step_ms": round(per[0] * 1e3, 1), "plain_step_ms": round(plain * 1e3, 2),
                     "mean_step_ms": round(sum(per) / 10 * 1e3, 2)}
        if name == "kfac":
            out[name]["plain_alg_tflops"] = round(flops / plain / 1e12, 2)
        if name == "kfac_newton":
            out[name]["inverse_method"] = "newton (coupled Newton, p = 1, fp32, batched)"
        del model, opt, X
        torch.cuda.empty_cache()
    if cpu:
        from pytorch_opt.ops import reference as ref

        g = torch.Generator().manual_seed(1)
        A = torch.randn(d + 1, d + 1, generator=g)
        G = torch.randn(d, d, generator=g)
        V = torch.randn(d, d + 1, generator=g)
        t_apply = timed(lambda: ref.precond_apply_two_sided(G, V, A))
        F = A.double() @ A.double().T
        t_eigh = timed(lambda: torch.linalg.eigh(F))
        plain_c = depth * t_apply
        refresh_c = plain_c + 2 * depth * t_eigh
        out["cpu"] = {"kfac_plain_step_ms": round(plain_c * 1e3, 1), "kfac_refresh_step_ms": round(refresh_c * 1e3, 1),
                      "kfac_mean_step_ms": round((refresh_c + 9 * plain_c) / 10 * 1e3, 1), "cores": cpu["threads"],
                      "kind": "port",
                      "sample": "pytorch_opt.ops.reference on CPU tensors: one (G·V)·A product of 2048x2049 and "
                                "one float64 eigh of 2049², scaled by 4 layers (and 8 eighs per refresh); mean "
                                "over one 10-step period"}
        out["kfac_speedup_vs_cpu"] = round(out["cpu"]["kfac_mean_step_ms"] / out["kfac"]["mean_step_ms"], 1)
        out["kfac_newton_speedup_vs_cpu"] = round(out["cpu"]["kfac_mean_step_ms"] / out["kfac_newton"]["mean_step_ms"], 1)
    return out


# ------------------------------------------------------------ HBM traffic

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "ns5_bf16_traffic.json")
COPY_BYTES = 1 << 30  # calibration copy: 1 GiB read + 1 GiB written


def kernel_probe(torch, ops, hip, dev, which):
    """A bounded run of one kernel family, for rocprofv3 (no timing output):
    factors  fp32 Kronecker update of G 4096² (beta 0.95) x10 and the K-FAC
             Gram of bf16 A 16384x4096 into fp32 x10;
    roots    the config-4 fp32 coupled-Newton roots at n = 1024, 2048, 4096
             (100 iterations each), twice;
    ns5      the headline step (32 x 4096² + 32 x 4096x11008 bf16) x3 and one
             4096² matrix x10;
    ns5-single  one 4096² bf16 matrix back to back for 15 s (board power
             and clock sampled beside it);
    shampoo  the fp32 2048² work of a plain Shampoo step on the 48
             attention matrices: the batched factor update (48 x (L, R),
             beta 0.999) x10, the two-sided apply L·G·R as one batched call
             over the stacked 48 x10, and as 48 single calls (the harness's
             per-parameter form) x2;
    optimizer  the config-5 Muon step and the Shampoo step (its arm of the
             set) on seeded gradients, 4 steps each (Shampoo's step 0
             refreshes the roots, steps 1-3 are plain)."""
    if which == "factors":
        g = torch.Generator(device=dev).manual_seed(2)
        G = 1e-2 * torch.randn(4096, 4096, generator=g, device=dev)
        L, R = G @ G.T, G.T @ G
        A = torch.randn(16384, 4096, generator=torch.Generator(device=dev).manual_seed(3), device=dev).bfloat16()
        F = torch.zeros(4096, 4096, device=dev)
        for _ in range(10):
            ops.kron_factor_update_(L, R, G, beta2=0.95)
        for _ in range(10):
            ops.gram_update_(F, A, beta=0.95, alpha=0.05 / 16384)
    elif which == "roots":
        for n in (1024, 2048, 4096):
            g = torch.Generator().manual_seed(4)
            Q, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
            lam = 10 ** (-6 * torch.rand(n, generator=torch.Generator().manual_seed(5), dtype=torch.float64))
            A = ((Q * lam) @ Q.T).float().to(dev)
            for _ in range(2):
                hip.inverse_matrix_root_iters(A, 4, 1e-6, "newton", False, 100, 1e-10)
    elif which == "ns5":
        inputs = [make_ns5_inputs(torch, b, r, c, s, dev) for b, r, c, s in SHAPES]
        for _ in range(3):
            for G in inputs:
                ops.newton_schulz_orthogonalize(G)
        single = inputs[0][:1].contiguous()
        for _ in range(10):
            ops.newton_schulz_orthogonalize(single)
    elif which == "ns5-single":
        single = make_ns5_inputs(torch, 1, 4096, 4096, SHAPES[0][3], dev)
        t_end = time.perf_counter() + 15.0
        while time.perf_counter() < t_end:
            for _ in range(100):
                ops.newton_schulz_orthogonalize(single)
            torch.cuda.synchronize()
    elif which == "shampoo":
        g = torch.Generator(device=dev).manual_seed(6)
        Gs = [1e-2 * torch.randn(2048, 2048, generator=g, device=dev) for _ in range(48)]
        Ls = [torch.eye(2048, device=dev) for _ in range(48)]
        Rs = [torch.eye(2048, device=dev) for _ in range(48)]
        for _ in range(10):
            ops.kron_factor_update_batched_(Ls, Rs, Gs, beta2=0.999)
        Gst = torch.stack(Gs)
        Lr = torch.stack(Ls) * (1.0 / Ls[0].norm())
        Rr = torch.stack(Rs) * (1.0 / Rs[0].norm())
        for _ in range(10):
            ops.precond_apply_two_sided(Lr, Gst, Rr)
        for _ in range(2):
            for i in range(48):
                ops.precond_apply_two_sided(Lr[i], Gs[i], Rr[i])
    elif which == "optimizer":
        from pytorch_opt import Muon, Shampoo

        mats, vecs = config5_shapes()
        kind = {n: k for n, _, k in mats}
        for arm in ("muon", "shampoo"):
            P = config5_params(torch, dev)
            rest = [P[n] for n, _ in vecs] + [P["emb"]]
            if arm == "muon":
                opt = Muon([{"params": [P[n] for n, _, _ in mats]}, {"params": rest, "use_muon": False}], lr=0.02)
            else:
                attn = [P[n] for n, _, _ in mats if kind[n] == "attn"]
                mlp = [P[n] for n, _, _ in mats if kind[n] == "mlp"]
                opt = Shampoo([{"params": attn}, {"params": mlp + rest, "use_preconditioner": False, "lr": 3e-4}],
                              max_preconditioner_dim=4096, precondition_frequency=20, graft="adagrad")
            for t in range(4):
                set_grads(torch, P, t, dev)
                opt.step()
            torch.cuda.synchronize()
            del P, opt
            torch.cuda.empty_cache()
    else:
        raise SystemExit(f"unknown probe {which!r}")
    torch.cuda.synchronize()
    print(f"probe {which} done", flush=True)


def traffic_probe(torch, ops, dev):
    """One NS5 step of the headline workload and a 1 GiB device copy, for
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs."""
    inputs = [make_ns5_inputs(torch, b, r, c, s, dev) for b, r, c, s in SHAPES]
    for G in inputs:
        ops.newton_schulz_orthogonalize(G)
    x = torch.ones(COPY_BYTES // 4, device=dev)
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    print("traffic probe done", flush=True)


def digest_traffic(fetch_csv, write_csv):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the ns5_update kernel,
    scaled by what the counters read for the 1 GiB copy."""
    import csv

    def per_kernel(path, counter):
        rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
        upd = [float(r["Counter_Value"]) for r in rows if "EpiNsUpdate" in r["Kernel_Name"]
               and "Tile<256" in r["Kernel_Name"].replace("TileILi256", "Tile<256")]
        # the 1 GiB same-dtype copy runs as the runtime's copyBuffer blit
        copy = [float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]]
        return upd, copy

    fu, fc = per_kernel(fetch_csv, "FETCH_SIZE")
    wu, wc = per_kernel(write_csv, "WRITE_SIZE")
    f_scale = COPY_BYTES / (max(fc) * 1024.0)
    w_scale = COPY_BYTES / (max(wc) * 1024.0)
    fetch = sum(fu) / len(fu) * 1024.0 * f_scale
    write = sum(wu) / len(wu) * 1024.0 * w_scale
    out = {"kernel": "ns5_update", "launches": len(fu), "fetch_bytes_per_launch": int(fetch),
           "write_bytes_per_launch": int(write), "traffic_bytes_per_launch": int(fetch + write),
           "copy_fetch_kib": max(fc), "copy_write_kib": max(wc), "fetch_scale": round(f_scale, 4),
           "write_scale": round(w_scale, 4)}
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def load_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


# ------------------------------------------------------------ main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="headline only (no factors/roots/optimizer)")
    ap.add_argument("--opt-steps", type=int, default=40)
    ap.add_argument("--traffic-probe", action="store_true", help="one NS5 step + 1 GiB copy, for PMC runs")
    ap.add_argument("--probe", choices=("factors", "roots", "ns5", "ns5-single", "shampoo", "optimizer"),
                    help="a bounded run of one kernel family for rocprofv3 or a power sampler, no timing")
    ap.add_argument("--digest-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write the ns5_update HBM traffic summary from two PMC runs")
    args = ap.parse_args()
    if args.digest_traffic:
        digest_traffic(*args.digest_traffic)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(matrices shard by whole matrices across GPUs; see the design notes).", file=sys.stderr)
        sys.exit(2)

    import torch

    from pytorch_opt import ops

    if not ops.load_native():
        raise RuntimeError("libpytorch_opt_hip.so did not load; run __graft_entry__.build()")
    ops.set_backend("native")
    hip = ops._NATIVE
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cpu = None if (args.no_cpu_baseline or args.probe or args.traffic_probe) else cpu_setup(torch)
    if args.traffic_probe:
        traffic_probe(torch, ops, dev)
        return
    if args.probe:
        kernel_probe(torch, ops, hip, dev, args.probe)
        return
    inputs = [make_ns5_inputs(torch, b, r, c, s, dev) for b, r, c, s in SHAPES]
    torch.cuda.synchronize()

    def step():
        return [ops.newton_schulz_orthogonalize(G) for G in inputs]

    for _ in range(args.warmup):
        step()
    # the timed region: no instrumentation
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        outs = step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    del outs
    # a second pass of the same steps with every MFMA launch bracketed by HIP
    # events on its stream: the per-kernel split and the roofline line
    hip.prof_reset()
    hip.prof_enable(True)
    for _ in range(args.steps):
        outs = step()
    torch.cuda.synchronize()
    hip.prof_enable(False)
    del outs

    ms_per_step = wall * 1e3 / args.steps
    flops_step = sum(b * ns5_flops(r, c) for b, r, c, _ in SHAPES)
    value = flops_step / (ms_per_step / 1e3) / 1e12
    kinds = {}
    for kind in ("ns5_gram", "ns5_square", "ns5_update"):
        ms, launches = hip.prof_query(kind)
        fl = args.steps * 5 * sum(b * ns5_kernel_flops(kind, r, c) for b, r, c, _ in SHAPES)
        kinds[kind] = {"ms_total": round(ms, 3), "launches": launches, "avg_ms": round(ms / max(launches, 1), 4),
                       "alg_flops_per_launch": fl // max(launches, 1),
                       "tflops": round(fl / (ms / 1e3) / 1e12, 2) if ms > 0 else None}
    dom = max(kinds, key=lambda k: kinds[k]["ms_total"])
    achieved = kinds[dom]["tflops"]

    single = inputs[0][:1].contiguous()
    single_ms = gpu_ms_per_call(torch, lambda: ops.newton_schulz_orthogonalize(single))
    single_tflops = ns5_flops(4096, 4096) / (single_ms / 1e3) / 1e12

    cpu_line = cpu_baseline_ns5(torch, inputs, cpu) if cpu else None
    del inputs
    torch.cuda.empty_cache()

    line = {
        "metric": "NS5 TFLOP/s (algorithmic, LAWN-41) on 32x4096^2 + 32x4096x11008 bf16, 5 iterations",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1e-3) gradients folded into Nesterov momentum (beta 0.95, 3 steps)",
        "config": {"workload": "batched NS5 bf16: 32 x 4096x4096 + 32 x 4096x11008, 5 quintic iterations",
                   "alg_flops_per_step": flops_step, "pct_bf16_mfma_peak": round(100 * value / PEAK["bf16"], 2)},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": PEAK["bf16"], "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK["bf16"], 4), "traffic": load_traffic(),
                     "traffic_source": "not measured in this run: bytes per ns5_update launch read from "
                                       "profiles/ns5_bf16_traffic.json, the digest of two rocprofv3 --pmc passes "
                                       "(FETCH_SIZE, WRITE_SIZE) of bench.py --traffic-probe scaled by a 1 GiB copy"},
        "kernels": kinds,
        "single_4096": {"ms": round(single_ms, 3), "tflops": round(single_tflops, 2),
                        "pct_bf16_mfma_peak": round(100 * single_tflops / PEAK["bf16"], 2)},
        "cpu_baseline": cpu_line,
    }
    if not args.no_extras:
        line["factors"] = bench_factors(torch, ops, hip, dev, cpu)
        line["roots"] = bench_roots(torch, hip, dev, cpu)
        line["optimizer"] = bench_optimizer(torch, ops, hip, dev, args.opt_steps, cpu)
        line["kfac"] = bench_kfac(torch, dev, cpu)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
