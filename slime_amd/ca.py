"""Python host mirror of the reference's pseudopod interface over the C ABI.

``Pseudopod`` follows ``ModelProtocol`` (slime/proto/model.cu:5-14): ``forward``
advances the CA, ``effective_rank`` and ``coherence`` score a history of states,
and ``fitness`` multiplies them (slime/kernels/warp_ca.cu:219). Device memory and
streams come from PyTorch; all arithmetic runs in ``libslime_ca.so``.

State tensors are CUDA tensors of shape [B, G, G, H*D] (channels-last), dtype
float32 or bfloat16 to match the handle.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

_DTYPES = {"fp32": _lib.SLIME_F32, "bf16": _lib.SLIME_BF16}


def _torch():
    import torch  # deferred: importing torch is slow and only needed for device memory
    return torch


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream=None) -> ctypes.c_void_p:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


class Pseudopod:
    """One multi-head neural-CA engine (a ``slime_ca`` handle).

    ``pvi_chain``: 0 computes P, I and V from the state; 1 chains them (I from P,
    V from I, slime/core/pseudopod.cu:98-119); 2 chains them with P from the 3x3
    neighbourhood sum of the state, the perception of multi_head_ca_kernel
    (slime/core/pseudopod.cu:62-91, toroidal here).

    ``growth_fn``: 0 the bell growth (failed_attempts/warp_ca.cu:49-56), 1 the
    Gaussian (failed_attempts/pseudopod.cu:46-48), 2 the shipped U exp(-U^2)
    (slime/core/pseudopod.cu:183). ``conservation``: 0 per (batch, head), 1 per
    (cell, head) first, as the shipped kernel renormalises
    (slime/core/pseudopod.cu:160-165,196-203)."""

    def __init__(self, B: int, G: int, H: int = 8, D: int = 64, dtype: str = "bf16",
                 dt: float = 0.1, growth_per_cell: bool = False, pods: int = 1,
                 pvi_chain: int = 0, growth_fn: int = 0, conservation: int = 0):
        if dtype not in _DTYPES:
            raise ValueError(f"dtype must be one of {sorted(_DTYPES)}")
        self.lib = _lib.load()
        self.B, self.G, self.H, self.D = B, G, H, D
        self.C = H * D
        self.dtype = dtype
        self.pods = pods
        self.growth_per_cell = growth_per_cell
        cfg = _lib.Config(B, G, H, D, _DTYPES[dtype], dt, int(growth_per_cell), pods,
                          int(pvi_chain), int(growth_fn), int(conservation))
        handle = ctypes.c_void_p()
        _lib.check(self.lib.slime_ca_create(ctypes.byref(cfg), ctypes.byref(handle)))
        self._h = handle
        self._keep = None

    # -- lifetime -------------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self.lib.slime_ca_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- helpers --------------------------------------------------------------------
    @property
    def torch_dtype(self):
        torch = _torch()
        return torch.bfloat16 if self.dtype == "bf16" else torch.float32

    @property
    def state_shape(self) -> tuple:
        return (self.B, self.G, self.G, self.C)

    def empty_state(self):
        torch = _torch()
        return torch.empty(self.state_shape, dtype=self.torch_dtype, device="cuda")

    def _check_state(self, t, name: str) -> None:
        if tuple(t.shape) != self.state_shape or t.dtype != self.torch_dtype or not t.is_cuda \
                or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous CUDA {self.torch_dtype} tensor of "
                             f"shape {self.state_shape}, got {tuple(t.shape)} {t.dtype}")

    @property
    def uses_mfma(self) -> bool:
        return bool(self.lib.slime_ca_uses_mfma(self._h))

    # -- parameters (init_multihead_ca_kernel, slime/core/pseudopod.cu:386-444) -------
    def set_params(self, params: dict) -> None:
        """``params``: WP, WI, WV [pods,C,C]; K [pods,H,9]; mu, sigma [pods,H] or
        [pods,G,G,H]; M [pods,H,H] — host arrays, converted to fp32."""
        arrs = {k: np.ascontiguousarray(params[k], dtype=np.float32)
                for k in ("WP", "WI", "WV", "K", "mu", "sigma", "M")}
        C, H, pods = self.C, self.H, self.pods
        expect = {"WP": (pods, C, C), "WI": (pods, C, C), "WV": (pods, C, C),
                  "K": (pods, H, 9), "M": (pods, H, H)}
        g = (pods, self.G, self.G, H) if self.growth_per_cell else (pods, H)
        expect["mu"] = expect["sigma"] = g
        for k, shp in expect.items():
            if arrs[k].size != int(np.prod(shp)):
                raise ValueError(f"{k} has {arrs[k].size} elements, expected shape {shp}")
        p = _lib.Params(*[arrs[k].ctypes.data for k in ("WP", "WI", "WV", "K", "mu", "sigma", "M")])
        _lib.check(self.lib.slime_ca_set_params(self._h, ctypes.byref(p)))

    # -- the step ---------------------------------------------------------------------
    def project(self, x, stream=None):
        """S1 (multi_head_ca_kernel, slime/core/pseudopod.cu:41-131) -> (P, I, V)."""
        self._check_state(x, "x")
        P, I, V = self.empty_state(), self.empty_state(), self.empty_state()
        _lib.check(self.lib.slime_ca_project(self._h, _ptr(x), _ptr(P), _ptr(I), _ptr(V),
                                             _stream(stream)))
        return P, I, V

    def flow_lenia(self, x, P, I, V, out=None, stream=None):
        """S2-S7 on given projections (flow_lenia_dynamics_kernel + mix_heads_kernel)."""
        for t, n in ((x, "x"), (P, "P"), (I, "I"), (V, "V")):
            self._check_state(t, n)
        y = out if out is not None else self.empty_state()
        self._check_state(y, "out")
        _lib.check(self.lib.slime_ca_flow_lenia(self._h, _ptr(x), _ptr(P), _ptr(I), _ptr(V),
                                                _ptr(y), _stream(stream)))
        return y

    def forward(self, x, out=None, n_steps: int = 1, stream=None):
        """n_steps full CA steps (ModelProtocol::forward, slime/proto/model.cu:10)."""
        self._check_state(x, "x")
        y = out if out is not None else self.empty_state()
        self._check_state(y, "out")
        _lib.check(self.lib.slime_ca_step(self._h, _ptr(x), _ptr(y), int(n_steps),
                                          _stream(stream)))
        return y

    step = forward

    def mass(self):
        """Per-(b, head) input and conserved output mass of the last step, [B, H] fp64."""
        mi = np.empty((self.B, self.H), np.float64)
        mo = np.empty((self.B, self.H), np.float64)
        _lib.check(self.lib.slime_ca_mass(self._h, mi.ctypes.data_as(ctypes.c_void_p),
                                          mo.ctypes.data_as(ctypes.c_void_p)))
        return mi, mo

    # -- gradient (update_gradients, declared only: slime/proto/model.cu:7,13) ----------
    def backward(self, x, target, params: bool = True, stream=None):
        """One step from ``x`` and the gradient of L = mean((step(x) - target)^2).

        Returns ``(loss, grad_x, grads)``: the loss as a float, dL/dx as a float32
        CUDA tensor of the state's shape and, when ``params``, a dict of float32
        CUDA tensors WP, WI, WV, K, mu, sigma, M shaped as the parameters (else
        an empty dict). Parallel projections only."""
        torch = _torch()
        self._check_state(x, "x")
        self._check_state(target, "target")
        gx = torch.empty(self.state_shape, dtype=torch.float32, device="cuda")
        grads = {}
        if params:
            C, H, pods = self.C, self.H, self.pods
            g = (pods, self.G, self.G, H) if self.growth_per_cell else (pods, H)
            shapes = {"WP": (pods, C, C), "WI": (pods, C, C), "WV": (pods, C, C),
                      "K": (pods, H, 9), "mu": g, "sigma": g, "M": (pods, H, H)}
            grads = {k: torch.empty(v, dtype=torch.float32, device="cuda") for k, v in shapes.items()}
        gs = _lib.Grads(*[grads[k].data_ptr() if k in grads else None
                          for k in ("WP", "WI", "WV", "K", "mu", "sigma", "M")])
        loss = ctypes.c_double()
        _lib.check(self.lib.slime_ca_backward(self._h, _ptr(x), _ptr(target), _ptr(gx),
                                              ctypes.byref(gs), ctypes.byref(loss),
                                              _stream(stream)))
        return loss.value, gx, grads

    # -- fitness (slime/kernels/warp_ca.cu:178-226) -------------------------------------
    def fitness(self, hist, stream=None):
        """``hist``: [T, B, G, G, C] CUDA tensor -> (erank, coherence, fitness), [B, H] each."""
        torch = _torch()
        if hist.dim() != 5 or tuple(hist.shape[1:]) != self.state_shape \
                or hist.dtype != self.torch_dtype or not hist.is_contiguous():
            raise ValueError(f"hist must be [T, {', '.join(map(str, self.state_shape))}] "
                             f"{self.torch_dtype}")
        outs = [torch.empty((self.B, self.H), dtype=torch.float32, device="cuda")
                for _ in range(3)]
        _lib.check(self.lib.slime_ca_fitness(self._h, _ptr(hist), int(hist.shape[0]),
                                             *[_ptr(o) for o in outs], _stream(stream)))
        return tuple(outs)

    def rollout(self, hist, stream=None):
        """T-1 steps from ``hist[0]`` into ``hist`` ([T, B, G, G, C], in place), each state
        stored before its mass rescale (slime_ca_rollout). Returns the factors, a float64
        CUDA tensor [T, B, H]: state t = factor[t, b, h] * hist[t] over head h."""
        torch = _torch()
        if hist.dim() != 5 or tuple(hist.shape[1:]) != self.state_shape \
                or hist.dtype != self.torch_dtype or not hist.is_contiguous():
            raise ValueError(f"hist must be [T, {', '.join(map(str, self.state_shape))}] "
                             f"{self.torch_dtype}")
        scales = torch.empty((hist.shape[0], self.B, self.H), dtype=torch.float64, device="cuda")
        _lib.check(self.lib.slime_ca_rollout(self._h, _ptr(hist), int(hist.shape[0]), _ptr(scales),
                                             _stream(stream)))
        return scales

    def fitness_scaled(self, hist, scales, stream=None):
        """fitness of a history left by ``rollout``: (erank, coherence, fitness), [B, H] each."""
        torch = _torch()
        if hist.dim() != 5 or tuple(hist.shape[1:]) != self.state_shape \
                or hist.dtype != self.torch_dtype or not hist.is_contiguous():
            raise ValueError(f"hist must be [T, {', '.join(map(str, self.state_shape))}] "
                             f"{self.torch_dtype}")
        if tuple(scales.shape) != (hist.shape[0], self.B, self.H) or scales.dtype != torch.float64 \
                or not scales.is_contiguous():
            raise ValueError("scales must be a contiguous float64 tensor [T, B, H]")
        outs = [torch.empty((self.B, self.H), dtype=torch.float32, device="cuda")
                for _ in range(3)]
        _lib.check(self.lib.slime_ca_fitness_scaled(self._h, _ptr(hist), _ptr(scales),
                                                    int(hist.shape[0]), *[_ptr(o) for o in outs],
                                                    _stream(stream)))
        return tuple(outs)

    def effective_rank(self, hist, stream=None):
        return self.fitness(hist, stream)[0]

    def coherence(self, hist, stream=None):
        return self.fitness(hist, stream)[1]

    def jacobi_sweeps(self) -> np.ndarray:
        out = np.empty((self.B, self.H), np.int32)
        _lib.check(self.lib.slime_ca_fitness_sweeps(self._h, out.ctypes.data_as(ctypes.c_void_p)))
        return out

    # -- kernel timing ----------------------------------------------------------------
    def set_timing(self, enable: bool) -> None:
        """Record HIP events around each GEMM and stencil launch of ``forward``."""
        _lib.check(self.lib.slime_ca_set_timing(self._h, int(bool(enable))))

    def timings(self) -> dict:
        gms, sms = ctypes.c_double(), ctypes.c_double()
        gn, sn = ctypes.c_int(), ctypes.c_int()
        _lib.check(self.lib.slime_ca_timings(self._h, ctypes.byref(gms), ctypes.byref(gn),
                                             ctypes.byref(sms), ctypes.byref(sn)))
        return {"gemm_ms": gms.value, "gemm_launches": gn.value, "stencil_ms": sms.value,
                "stencil_launches": sn.value}

    # -- organism adapters (slime/core/organism.cu:691-743) -----------------------------
    def init_from_field(self, conc, stream=None):
        torch = _torch()
        conc = conc.to(device="cuda", dtype=torch.float32).contiguous()
        x = torch.empty((self.G, self.G, self.C), dtype=self.torch_dtype, device="cuda")
        _lib.check(self.lib.slime_ca_init_from_field(self._h, _ptr(conc), _ptr(x), _stream(stream)))
        return x

    def neural_ca_update(self, conc, ca_input, ca_output, erank_history, generation: int,
                         mass_buffer=None, stream=None):
        """One organism generation (neural_ca_update_kernel, slime/core/organism.cu:617-688)
        on a B = 1 handle: ``ca_input`` <- field, ``ca_output`` <- one step,
        ``conc`` <- mean over channels of ``ca_output`` (updated in place),
        ``erank_history[generation]`` <- mean per-head effective rank of ``ca_output``,
        ``mass_buffer`` (optional, [H] fp32) <- per-head conserved mass."""
        torch = _torch()
        shape = (self.G, self.G, self.C)
        for t, n in ((ca_input, "ca_input"), (ca_output, "ca_output")):
            if tuple(t.shape) != shape or t.dtype != self.torch_dtype or not t.is_cuda \
                    or not t.is_contiguous():
                raise ValueError(f"{n} must be a contiguous CUDA {self.torch_dtype} tensor of "
                                 f"shape {shape}")
        for t, n, shp in ((conc, "conc", (self.G, self.G)),
                          (erank_history, "erank_history", None),
                          (mass_buffer, "mass_buffer", (self.H,))):
            if t is None and n == "mass_buffer":
                continue
            if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous() \
                    or (shp is not None and tuple(t.shape) != shp):
                raise ValueError(f"{n} must be a contiguous CUDA float32 tensor"
                                 + (f" of shape {shp}" if shp else ""))
        if not 0 <= generation < erank_history.numel():
            raise ValueError(f"generation {generation} is outside erank_history")
        st = _lib.MultiHeadCAState(mass_buffer.data_ptr() if mass_buffer is not None else None,
                                   ca_input.data_ptr(), ca_output.data_ptr())
        _lib.check(self.lib.slime_neural_ca_update(self._h, ctypes.byref(st), _ptr(conc),
                                                   _ptr(erank_history), int(generation),
                                                   _stream(stream)))

    def field_from_state(self, x, stream=None):
        torch = _torch()
        conc = torch.empty((self.G, self.G), dtype=torch.float32, device="cuda")
        _lib.check(self.lib.slime_ca_field_from_state(self._h, _ptr(x), _ptr(conc), _stream(stream)))
        return conc

    def get_state(self, x, size=None):
        """The field of state ``x`` on the host (get_ca_state, slime/runtime.cu:479-504):
        the first ``size`` (default G*G) values of mean_c x, row-major, as float32."""
        n = self.G * self.G if size is None else int(size)
        out = np.empty(max(n, 0), dtype=np.float32)
        _lib.check(self.lib.slime_ca_get_state(self._h, _ptr(x), out.ctypes.data, n))
        return out
