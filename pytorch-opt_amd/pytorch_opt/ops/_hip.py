"""ctypes adapter from torch tensors to the C ABI of libpytorch_opt_hip.so.

``HipBackend`` is the object the dispatch layer stores in ``ops._NATIVE``.
Its methods take the exact positional forms the dispatch calls
(pytorch_opt/ops/__init__.py:61-62,70,76,83 in the reference) and turn
tensors into device pointers, extents, a dtype code, a torch-allocated
workspace and the current HIP stream. GPU tensors always run the HIP
kernels; a failing call raises RuntimeError with the library's message and
never falls back. CPU tensors take the pure-torch maths, as the reference's
compiled backend served CPU tensors through ATen.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import reference
from .reference import OpsArgumentError, ROOT_METHODS

_DTYPE_CODE = {torch.float32: 0, torch.float64: 1, torch.bfloat16: 2}

# Root methods that run the coupled Newton kernels on GPU tensors; "eigh"
# stays on torch.linalg.eigh (an eigendecomposition, not one of the kernels).
_NEWTON_METHODS = ("auto", "newton")

_c_size = ctypes.c_size_t
_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_dbl = ctypes.c_double
_c_ptr = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/pytorch_opt_hip.h
SIGNATURES = {
    "pto_last_error": (ctypes.c_char_p, []),
    "pto_version": (_c_int, []),
    "pto_runtime_version": (_c_int, []),
    "pto_ns5_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64]),
    "pto_ns5": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_dbl, _c_dbl, _c_dbl,
                         _c_dbl, _c_ptr, _c_size, _c_ptr]),
    "pto_ns5_noalloc": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_dbl, _c_dbl, _c_dbl,
                                 _c_dbl, _c_ptr]),
    "pto_kron_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64]),
    "pto_kron_factor_update": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_dbl, _c_ptr,
                                        _c_size, _c_ptr]),
    "pto_gram_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64, _c_int]),
    "pto_gram_update": (_c_int, [_c_ptr, _c_int, _c_ptr, _c_int, _c_i64, _c_i64, _c_int, _c_dbl, _c_dbl,
                                 _c_ptr, _c_size, _c_ptr]),
    "pto_inverse_root_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64]),
    "pto_inverse_root": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_dbl, _c_i64,
                                  _c_dbl, _c_ptr, _c_size, ctypes.POINTER(_c_i64), _c_ptr]),
    "pto_inverse_root_each_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64]),
    "pto_inverse_root_each": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_dbl, _c_i64,
                                       _c_dbl, _c_ptr, _c_size, ctypes.POINTER(_c_i64), _c_ptr]),
    "pto_precond_apply_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64]),
    "pto_precond_apply": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_ptr, _c_size,
                                   _c_ptr]),
    "pto_two_sided_product_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64]),
    "pto_two_sided_product": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_int, _c_int,
                                       _c_ptr, _c_size, _c_ptr]),
    "pto_two_sided_product_batched_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "pto_two_sided_product_batched": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64,
                                               _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr, _c_size, _c_ptr]),
    "pto_kron_batched_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64]),
    "pto_kron_factor_update_batched": (_c_int, [ctypes.POINTER(_c_ptr), ctypes.POINTER(_c_ptr), _c_ptr, _c_int, _c_i64,
                                                _c_i64, _c_i64, _c_dbl, _c_ptr, _c_size, _c_ptr]),
    "pto_adamw_workspace_bytes": (_c_size, []),
    "pto_adamw_step": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_dbl, _c_dbl, _c_dbl, _c_dbl,
                                _c_dbl, _c_i64, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "pto_muon_update_workspace_bytes": (_c_size, []),
    "pto_muon_momentum": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_dbl, _c_int, _c_ptr]),
    "pto_muon_update": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_dbl, _c_dbl, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "pto_shampoo_graft_workspace_bytes": (_c_size, []),
    "pto_shampoo_graft": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_dbl, _c_dbl, _c_dbl,
                                   _c_dbl, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "pto_prof_enable": (_c_int, [_c_int]),
    "pto_prof_reset": (_c_int, []),
    "pto_prof_query": (_c_int, [ctypes.c_char_p, ctypes.POINTER(_c_dbl), ctypes.POINTER(_c_i64)]),
}


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _overlaps(a: torch.Tensor, b: torch.Tensor) -> bool:
    if a.device != b.device or a.numel() == 0 or b.numel() == 0:
        return False
    a0, b0 = a.data_ptr(), b.data_ptr()
    a1 = a0 + a.numel() * a.element_size()
    b1 = b0 + b.numel() * b.element_size()
    return a0 < b1 and b0 < a1


class HipBackend:
    """The compiled backend object: same call forms as the reference's _NATIVE."""

    def __init__(self, path: str):
        self.path = path
        self._lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(self._lib, name)
            fn.restype = res
            fn.argtypes = args
        self.version = self._lib.pto_version()

    # ------------------------------------------------------------ plumbing
    def _check(self, rc: int, what: str) -> None:
        if rc != 0:
            msg = self._lib.pto_last_error().decode(errors="replace")
            raise RuntimeError(f"{what}: {msg} (status {rc})")

    @staticmethod
    def _stream(dev: torch.device) -> ctypes.c_void_p:
        return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    @staticmethod
    def _workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
        return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)

    # ------------------------------------------------------------ ops
    def newton_schulz_orthogonalize(self, G, steps, a, b, c, eps):
        if G.dim() < 2:
            raise OpsArgumentError("newton_schulz_orthogonalize expects a matrix (ndim >= 2)")
        if not G.is_cuda:
            return reference.newton_schulz_orthogonalize(G, steps, (a, b, c), eps)
        if G.dtype not in _DTYPE_CODE:  # e.g. float16: the float32 path, cast back
            return self.newton_schulz_orthogonalize(G.float(), steps, a, b, c, eps).to(G.dtype)
        Gc = G.contiguous()
        rows, cols = Gc.shape[-2], Gc.shape[-1]
        batch = math.prod(Gc.shape[:-2])
        out = torch.empty_like(Gc)
        code = _DTYPE_CODE[Gc.dtype]
        with torch.cuda.device(Gc.device):
            nbytes = self._lib.pto_ns5_workspace_bytes(code, batch, rows, cols)
            ws = self._workspace(nbytes, Gc.device)
            rc = self._lib.pto_ns5(_ptr(Gc), _ptr(out), code, batch, rows, cols, max(int(steps), 0),
                                   float(a), float(b), float(c), float(eps), _ptr(ws), nbytes,
                                   self._stream(Gc.device))
        self._check(rc, "newton_schulz_orthogonalize")
        return out

    def newton_schulz_orthogonalize_into(self, G, out, steps, a, b, c, eps):
        """NS5 of a contiguous GPU tensor G into the caller's `out` (same shape
        and dtype) through pto_ns5_noalloc: nothing is allocated, the library's
        static per-GPU scratch serves as the workspace."""
        if G.dim() < 2:
            raise OpsArgumentError("newton_schulz_orthogonalize expects a matrix (ndim >= 2)")
        if not (G.is_cuda and out.is_cuda and G.is_contiguous() and out.is_contiguous()):
            raise OpsArgumentError("newton_schulz_orthogonalize_into: contiguous GPU tensors only")
        if out.shape != G.shape or out.dtype != G.dtype or G.dtype not in _DTYPE_CODE:
            raise OpsArgumentError("newton_schulz_orthogonalize_into: out must match G (float32, float64, bfloat16)")
        if _overlaps(G, out) and G.data_ptr() != out.data_ptr():
            raise OpsArgumentError("newton_schulz_orthogonalize_into: out must be G itself or not overlap it")
        rows, cols = G.shape[-2], G.shape[-1]
        batch = math.prod(G.shape[:-2])
        with torch.cuda.device(G.device):
            rc = self._lib.pto_ns5_noalloc(_ptr(G), _ptr(out), _DTYPE_CODE[G.dtype], batch, rows, cols,
                                           max(int(steps), 0), float(a), float(b), float(c), float(eps),
                                           self._stream(G.device))
        self._check(rc, "newton_schulz_orthogonalize_into")
        return out

    def kron_factor_update_(self, L, R, G, beta2):
        if G.dim() != 2:
            raise OpsArgumentError(f"G must be 2D, got shape {tuple(G.shape)}")
        if not (G.is_cuda and L.is_cuda and R.is_cuda):
            reference.kron_factor_update_(L, R, G, beta2)
            return
        m, n = G.shape
        if tuple(L.shape) != (m, m) or tuple(R.shape) != (n, n):
            raise OpsArgumentError(f"kron_factor_update_: L {tuple(L.shape)} and R {tuple(R.shape)} "
                                   f"do not match G {tuple(G.shape)}")
        if L.dtype != R.dtype:
            raise OpsArgumentError("kron_factor_update_: L and R must share a dtype")
        work = L.dtype if L.dtype in _DTYPE_CODE else torch.float32
        Lw = L if (L.dtype == work and L.is_contiguous()) else L.to(work).contiguous()
        Rw = R if (R.dtype == work and R.is_contiguous()) else R.to(work).contiguous()
        Gw = G.to(work).contiguous()
        if _overlaps(Gw, Lw) or _overlaps(Gw, Rw):
            Gw = Gw.clone()  # the update reads G after writing L/R
        code = _DTYPE_CODE[work]
        with torch.cuda.device(Gw.device):
            nbytes = self._lib.pto_kron_workspace_bytes(code, m, n)
            ws = self._workspace(nbytes, Gw.device)
            rc = self._lib.pto_kron_factor_update(_ptr(Lw), _ptr(Rw), _ptr(Gw), code, m, n, float(beta2),
                                                  _ptr(ws), nbytes, self._stream(Gw.device))
        self._check(rc, "kron_factor_update_")
        if Lw is not L:
            L.copy_(Lw)
        if Rw is not R:
            R.copy_(Rw)

    # matrices per launch of the batched factor update (its epilogue's
    # table), and the bytes of stacked gradients per launch: the stack and
    # the workspace (Gᵀ and, for unpadded widths, a padded G) are transient
    # copies of about that size each
    KRON_BATCH = 64
    KRON_BATCH_BYTES = 1 << 30

    def kron_factor_update_batched_(self, Ls, Rs, Gs, beta2):
        """kron_factor_update_ on each (L, R, G) of same-shape lists, one launch
        per side for up to KRON_BATCH matrices and KRON_BATCH_BYTES of
        gradients; in float32 and float64 each factor gets the bits the
        single call gives it (bfloat16 may differ in the last bits: the tile
        depends on the batch). The gradients of a launch are stacked into
        one tensor."""
        k = len(Gs)
        if not (len(Ls) == len(Rs) == k):
            raise OpsArgumentError("kron_factor_update_batched_: L, R and G lists differ in length")
        if k == 0:
            return
        m, n = Gs[0].shape if Gs[0].dim() == 2 else (None, None)
        if m is None or any(G.dim() != 2 or tuple(G.shape) != (m, n) for G in Gs):
            raise OpsArgumentError("kron_factor_update_batched_: every G must be 2D with one shape")
        dev, dt = Ls[0].device, Ls[0].dtype
        same = all(t.device == dev and t.dtype == dt and t.is_contiguous() for t in list(Ls) + list(Rs))
        if (not same or dt not in _DTYPE_CODE or not dev.type == "cuda"
                or any(tuple(L.shape) != (m, m) for L in Ls) or any(tuple(R.shape) != (n, n) for R in Rs)):
            for L, R, G in zip(Ls, Rs, Gs):  # mixed layouts: one call each
                self.kron_factor_update_(L, R, G, beta2)
            return
        code = _DTYPE_CODE[dt]
        g_bytes = max(m * n * (torch.finfo(dt).bits // 8), 1)
        per = max(1, min(self.KRON_BATCH, self.KRON_BATCH_BYTES // g_bytes))
        for c0 in range(0, k, per):
            cl, cr = Ls[c0:c0 + per], Rs[c0:c0 + per]
            Gst = torch.stack([G.to(device=dev, dtype=dt) for G in Gs[c0:c0 + per]])
            b = len(cl)
            lt = (_c_ptr * b)(*[t.data_ptr() for t in cl])
            rt = (_c_ptr * b)(*[t.data_ptr() for t in cr])
            with torch.cuda.device(dev):
                nbytes = self._lib.pto_kron_batched_workspace_bytes(code, b, m, n)
                ws = self._workspace(nbytes, dev)
                rc = self._lib.pto_kron_factor_update_batched(lt, rt, _ptr(Gst), code, b, m, n, float(beta2),
                                                              _ptr(ws), nbytes, self._stream(dev))
            self._check(rc, "kron_factor_update_batched_")

    @staticmethod
    def newton_for(method: str) -> bool:
        """Whether `method` runs the coupled Newton kernels on GPU tensors."""
        return method in _NEWTON_METHODS

    def inverse_matrix_root(self, A, p, damping, method, root_f64, max_iter, tol):
        return self.inverse_matrix_root_iters(A, p, damping, method, root_f64, max_iter, tol)[0]

    def inverse_matrix_root_iters(self, A, p, damping, method, root_f64, max_iter, tol):
        """inverse_matrix_root plus the number of Newton iterations run."""
        if int(p) != p or p < 1:
            raise OpsArgumentError(f"p must be a positive integer, got {p}")
        if method not in ROOT_METHODS:
            raise OpsArgumentError(f"method must be one of {ROOT_METHODS}, got {method!r}")
        root_dtype = torch.float64 if root_f64 else torch.float32
        if not A.is_cuda or not self.newton_for(method):
            # eigendecomposition is not one of the kernels here: torch's eigh
            return reference.inverse_matrix_root_with_iters(A, p, damping, method, root_dtype, max_iter, tol)
        if A.dim() < 2 or A.shape[-1] != A.shape[-2]:
            raise OpsArgumentError(f"inverse_matrix_root expects square matrices, got {tuple(A.shape)}")
        if A.dtype not in _DTYPE_CODE:
            out, iters = self.inverse_matrix_root_iters(A.float(), p, damping, method, root_f64, max_iter, tol)
            return out.to(A.dtype), iters
        Ac = A.contiguous()
        n = Ac.shape[-1]
        batch = math.prod(Ac.shape[:-2])
        out = torch.empty_like(Ac)
        code = _DTYPE_CODE[Ac.dtype]
        iters = _c_i64(0)
        with torch.cuda.device(Ac.device):
            nbytes = self._lib.pto_inverse_root_workspace_bytes(int(bool(root_f64)), batch, n, max(int(max_iter), 0))
            ws = self._workspace(nbytes, Ac.device)
            rc = self._lib.pto_inverse_root(_ptr(Ac), _ptr(out), code, int(bool(root_f64)), batch, n, int(p),
                                            float(damping), max(int(max_iter), 0), float(tol), _ptr(ws), nbytes,
                                            ctypes.byref(iters), self._stream(Ac.device))
        self._check(rc, "inverse_matrix_root")
        return out, int(iters.value)

    def inverse_matrix_root_each(self, A, p, damping, root_f64, max_iter, tol):
        """Coupled-Newton roots of a stack A [k, n, n] of independent matrices,
        each by its own stop rule (what k separate inverse_matrix_root calls
        return), in one launch sequence. Returns (roots, iterations per matrix)."""
        if int(p) != p or p < 1:
            raise OpsArgumentError(f"p must be a positive integer, got {p}")
        if A.dim() != 3 or A.shape[-1] != A.shape[-2]:
            raise OpsArgumentError(f"inverse_matrix_root_each expects [k, n, n], got {tuple(A.shape)}")
        if not A.is_cuda:
            outs = [reference.inverse_matrix_root_with_iters(a, p, damping, "newton",
                                                             torch.float64 if root_f64 else torch.float32,
                                                             max_iter, tol) for a in A]
            return torch.stack([o for o, _ in outs]), [i for _, i in outs]
        if A.dtype not in _DTYPE_CODE:
            out, iters = self.inverse_matrix_root_each(A.float(), p, damping, root_f64, max_iter, tol)
            return out.to(A.dtype), iters
        Ac = A.contiguous()
        k, n = Ac.shape[0], Ac.shape[-1]
        out = torch.empty_like(Ac)
        code = _DTYPE_CODE[Ac.dtype]
        iters = (_c_i64 * max(k, 1))()
        with torch.cuda.device(Ac.device):
            nbytes = self._lib.pto_inverse_root_each_workspace_bytes(int(bool(root_f64)), k, n,
                                                                     max(int(max_iter), 0))
            ws = self._workspace(nbytes, Ac.device)
            rc = self._lib.pto_inverse_root_each(_ptr(Ac), _ptr(out), code, int(bool(root_f64)), k, n, int(p),
                                                 float(damping), max(int(max_iter), 0), float(tol), _ptr(ws),
                                                 nbytes, iters, self._stream(Ac.device))
        self._check(rc, "inverse_matrix_root_each")
        return out, [int(iters[i]) for i in range(k)]

    def precond_apply_two_sided(self, L_root, G, R_root):
        if not (L_root.is_cuda and G.is_cuda and R_root.is_cuda):
            return reference.precond_apply_two_sided(L_root, G, R_root)
        return self._two_sided(L_root, G, R_root, False, False, "precond_apply_two_sided")

    def two_sided_product(self, A, X, B, transpose_a, transpose_b):
        if not (A.is_cuda and X.is_cuda and B.is_cuda):
            return reference.two_sided_product(A, X, B, transpose_a, transpose_b)
        return self._two_sided(A, X, B, bool(transpose_a), bool(transpose_b), "two_sided_product")

    def _two_sided(self, A, X, B, trans_a, trans_b, what):
        """op(A)·X·op(B) per matrix of the broadcast batch (square A and B)."""
        if A.dim() < 2 or X.dim() < 2 or B.dim() < 2:
            raise OpsArgumentError(f"{what} expects matrices")
        m, n = X.shape[-2], X.shape[-1]
        if A.shape[-2:] != (m, m) or B.shape[-2:] != (n, n):
            raise OpsArgumentError(f"{what}: shapes {tuple(A.shape)}, {tuple(X.shape)}, "
                                   f"{tuple(B.shape)} do not chain")
        out_dtype = torch.promote_types(torch.promote_types(A.dtype, X.dtype), B.dtype)
        work = out_dtype if out_dtype in _DTYPE_CODE else torch.float32
        lead = torch.broadcast_shapes(A.shape[:-2], X.shape[:-2], B.shape[:-2])
        if math.prod(lead) > 1:
            out = self._two_sided_batched(A.to(work), X.to(work), B.to(work), lead, m, n, trans_a, trans_b, what)
            return out if out.dtype == out_dtype else out.to(out_dtype)
        Ab = A.to(work).expand(*lead, m, m).reshape(-1, m, m)
        Xb = X.to(work).expand(*lead, m, n).reshape(-1, m, n)
        Bb = B.to(work).expand(*lead, n, n).reshape(-1, n, n)
        out = torch.empty(Xb.shape, dtype=work, device=X.device)
        code = _DTYPE_CODE[work]
        with torch.cuda.device(X.device):
            nbytes = self._lib.pto_two_sided_product_workspace_bytes(code, m, n)
            ws = self._workspace(nbytes, X.device)
            stream = self._stream(X.device)
            for i in range(out.shape[0]):
                Ai, Xi, Bi = Ab[i].contiguous(), Xb[i].contiguous(), Bb[i].contiguous()
                if trans_a or trans_b:
                    rc = self._lib.pto_two_sided_product(_ptr(Ai), _ptr(Xi), _ptr(Bi), _ptr(out[i]), code, m, n,
                                                         int(trans_a), int(trans_b), _ptr(ws), nbytes, stream)
                else:
                    rc = self._lib.pto_precond_apply(_ptr(Ai), _ptr(Xi), _ptr(Bi), _ptr(out[i]), code, m, n,
                                                     _ptr(ws), nbytes, stream)
                self._check(rc, what)
        out = out.reshape(*lead, m, n)
        return out if out.dtype == out_dtype else out.to(out_dtype)

    # workspace per batched call (packed copies and the intermediate)
    two_sided_batch_bytes = 4 << 30

    def _two_sided_batched(self, A, X, B, lead, m, n, trans_a, trans_b, what):
        """op(A)·X·op(B) over the broadcast batch `lead`, one launch per
        product per chunk; a factor whose leading dims are all 1 is shared
        (stride 0) instead of copied per matrix."""
        batch = math.prod(lead)

        def operand(T, r, c):
            if math.prod(T.shape[:-2]) == 1:
                return T.reshape(r, c).contiguous(), 0
            return T.expand(*lead, r, c).reshape(batch, r, c).contiguous(), r * c

        Ab, sa = operand(A, m, m)
        Xb, sx = operand(X, m, n)
        Bb, sb = operand(B, n, n)
        out = torch.empty(batch, m, n, dtype=X.dtype, device=X.device)
        code = _DTYPE_CODE[X.dtype]
        with torch.cuda.device(X.device):
            per = max(1, self._lib.pto_two_sided_product_batched_workspace_bytes(code, 1, m, n, 0, 0))
            chunk = max(1, min(65535, self.two_sided_batch_bytes // per))
            stream = self._stream(X.device)
            for s in range(0, batch, chunk):
                nb = min(chunk, batch - s)
                nbytes = self._lib.pto_two_sided_product_batched_workspace_bytes(code, nb, m, n, int(sa == 0),
                                                                                 int(sb == 0))
                ws = self._workspace(nbytes, X.device)
                pa = Ab[s] if sa else Ab
                px = Xb[s] if sx else Xb
                pb = Bb[s] if sb else Bb
                rc = self._lib.pto_two_sided_product_batched(_ptr(pa), _ptr(px), _ptr(pb), _ptr(out[s]), code, nb, m,
                                                             n, sa, sx, sb, int(trans_a), int(trans_b), _ptr(ws),
                                                             nbytes, stream)
                self._check(rc, what)
        return out.reshape(*lead, m, n)

    @staticmethod
    def _fusable(*ts) -> bool:
        """Same device (a GPU), dtype with a kernel, element count, and
        contiguous: the fused elementwise kernels' preconditions."""
        t0 = ts[0]
        return (all(t.is_cuda and t.device == t0.device for t in ts) and t0.dtype in _DTYPE_CODE
                and all(t.dtype == t0.dtype and t.numel() == t0.numel() and t.is_contiguous() for t in ts))

    def muon_momentum_(self, buf, g, u, momentum, nesterov):
        if buf.shape != g.shape or not self._fusable(buf, g, u):
            return reference.muon_momentum_(buf, g, u, momentum, nesterov)
        with torch.cuda.device(buf.device):
            rc = self._lib.pto_muon_momentum(_ptr(buf), _ptr(g), _ptr(u), _DTYPE_CODE[buf.dtype], buf.numel(),
                                             float(momentum), int(bool(nesterov)), self._stream(buf.device))
        self._check(rc, "muon_momentum_")
        return u

    def muon_update_(self, p, O, decay, neg_lr):
        if not self._fusable(p, O):
            return reference.muon_update_(p, O, decay, neg_lr)
        sq = torch.empty((), dtype=torch.float64, device=p.device)
        with torch.cuda.device(p.device):
            nbytes = self._lib.pto_muon_update_workspace_bytes()
            ws = self._workspace(nbytes, p.device)
            rc = self._lib.pto_muon_update(_ptr(p), _ptr(O), _DTYPE_CODE[p.dtype], p.numel(), float(decay),
                                           float(neg_lr), _ptr(sq), _ptr(ws), nbytes, self._stream(p.device))
        self._check(rc, "muon_update_")
        return sq

    def shampoo_graft_(self, p, g, acc, P, buf, diag_eps, momentum, decay, neg_lr):
        ts = (p, g, acc, P) + ((buf,) if buf is not None else ())
        if (buf is not None) != bool(momentum) or g.shape != acc.shape or not self._fusable(*ts):
            return reference.shampoo_graft_(p, g, acc, P, buf, diag_eps, momentum, decay, neg_lr)
        ratio = torch.empty((), dtype=p.dtype, device=p.device)
        with torch.cuda.device(p.device):
            nbytes = self._lib.pto_shampoo_graft_workspace_bytes()
            ws = self._workspace(nbytes, p.device)
            rc = self._lib.pto_shampoo_graft(_ptr(p), _ptr(g), _ptr(acc), _ptr(P),
                                             _ptr(buf) if buf is not None else None, _DTYPE_CODE[p.dtype],
                                             p.numel(), float(diag_eps), float(momentum), float(decay),
                                             float(neg_lr), _ptr(ratio), _ptr(ws), nbytes, self._stream(p.device))
        self._check(rc, "shampoo_graft_")
        return ratio

    def adamw_step_(self, p, g, m, v, lr, weight_decay, beta1, beta2, eps, step, return_update_sq):
        tensors = (p, g, m, v)
        if not all(t.is_cuda for t in tensors):
            return reference.adamw_step_(p, g, m, v, lr, weight_decay, (beta1, beta2), eps, step, return_update_sq)
        if any(t.shape != p.shape or t.dtype != p.dtype for t in tensors):
            raise OpsArgumentError("adamw_step_: p, grad and both moments must share shape and dtype")
        if p.dtype not in _DTYPE_CODE:
            # float16 has no kernel here: torch's own elementwise ops, on the GPU, in the reference's order
            return reference.adamw_step_(p, g, m, v, lr, weight_decay, (beta1, beta2), eps, step, return_update_sq)
        work = [t if t.is_contiguous() else t.contiguous() for t in tensors]
        sq = torch.empty((), dtype=torch.float64, device=p.device) if return_update_sq else None
        with torch.cuda.device(p.device):
            nbytes = self._lib.pto_adamw_workspace_bytes()
            ws = self._workspace(nbytes, p.device) if return_update_sq else None
            rc = self._lib.pto_adamw_step(_ptr(work[0]), _ptr(work[1]), _ptr(work[2]), _ptr(work[3]),
                                          _DTYPE_CODE[p.dtype], p.numel(), float(lr), float(weight_decay),
                                          float(beta1), float(beta2), float(eps), int(step),
                                          _ptr(sq) if sq is not None else None,
                                          _ptr(ws) if ws is not None else None, nbytes if ws is not None else 0,
                                          self._stream(p.device))
        self._check(rc, "adamw_step_")
        for dst, src in zip((p, m, v), (work[0], work[2], work[3])):
            if dst is not src:
                dst.copy_(src)
        return sq

    def gram_update_(self, F, X, beta, alpha, append_ones):
        if not (F.is_cuda and X.is_cuda):
            reference.gram_update_(F, X, beta, alpha, append_ones)
            return
        d = X.shape[-1]
        X2 = X.reshape(-1, d)
        dd = d + (1 if append_ones else 0)
        if tuple(F.shape) != (dd, dd):
            raise OpsArgumentError(f"gram_update_: F {tuple(F.shape)} does not match X̃ width {dd}")
        f_work = F.dtype if F.dtype in (torch.float32, torch.float64) else torch.float32
        x_work = X2.dtype if (X2.dtype == torch.bfloat16 and f_work == torch.float32) else f_work
        Fw = F if (F.dtype == f_work and F.is_contiguous()) else F.to(f_work).contiguous()
        Xw = X2.to(x_work).contiguous()
        if _overlaps(Xw, Fw) or Xw.data_ptr() % 16:  # bf16 X may be read in place: 16-byte aligned
            Xw = Xw.clone()
        fc, xc = _DTYPE_CODE[f_work], _DTYPE_CODE[x_work]
        rows = Xw.shape[0]
        with torch.cuda.device(Fw.device):
            nbytes = self._lib.pto_gram_workspace_bytes(xc, rows, d, int(bool(append_ones)))
            ws = self._workspace(nbytes, Fw.device)
            rc = self._lib.pto_gram_update(_ptr(Fw), fc, _ptr(Xw), xc, rows, d, int(bool(append_ones)),
                                           float(beta), float(alpha), _ptr(ws), nbytes, self._stream(Fw.device))
        self._check(rc, "gram_update_")
        if Fw is not F:
            F.copy_(Fw)

    # ------------------------------------------------------------ timing
    def prof_enable(self, on: bool) -> None:
        self._check(self._lib.pto_prof_enable(int(bool(on))), "prof_enable")

    def prof_reset(self) -> None:
        self._check(self._lib.pto_prof_reset(), "prof_reset")

    def prof_query(self, name: str):
        """(total milliseconds, launches) recorded for one kernel class."""
        ms, n = _c_dbl(0.0), _c_i64(0)
        self._check(self._lib.pto_prof_query(name.encode(), ctypes.byref(ms), ctypes.byref(n)), "prof_query")
        return ms.value, n.value
