"""torch.optim for the 'hip' device: Adam / AdamW (src/optim/adam.ts,
src/optim/adamw.ts) as one fused multi-tensor kernel per step, with no
device->host readback (the reference reads back 3-4 tensors per parameter
and updates in a JS loop, adam.ts:104-120), plus plain SGD.
"""
import ctypes

from . import _lib as L
from .tensor import Tensor, _before_write, _k_contiguous, capturing, zeros


class Optimizer:
    """Optimizer base (src/optim/optimizer.ts:19-72): param_groups built
    from a list of tensors or of {'params': [...], ...} dicts."""

    def __init__(self, params, defaults):
        self.defaults = dict(defaults)
        self.param_groups = []
        params = list(params)
        if params and isinstance(params[0], dict):
            for g in params:
                grp = dict(self.defaults)
                grp.update(g)
                grp["params"] = list(g["params"])
                grp.setdefault("initial_lr", grp["lr"])
                self.param_groups.append(grp)
        else:
            grp = dict(self.defaults)
            grp["params"] = params
            grp["initial_lr"] = grp["lr"]
            self.param_groups.append(grp)
        self.state = {}

    def zero_grad(self, set_to_none=True):
        for g in self.param_groups:
            for p in g["params"]:
                p.grad = None

    def step(self):
        raise NotImplementedError


def _opts(options, kwargs, defaults):
    o = dict(defaults)
    if options:
        o.update(options)
    o.update(kwargs)
    return o


class Adam(Optimizer):
    """Adam (src/optim/adam.ts:46-133): L2 weight decay added to the grad."""

    _decoupled = 0
    _default_wd = 0.0

    def __init__(self, params, options=None, **kwargs):
        o = _opts(options, kwargs, {"lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8,
                                    "weight_decay": self._default_wd, "amsgrad": False,
                                    "capturable": False})
        if o["amsgrad"]:
            raise NotImplementedError("AMSGrad not yet fully implemented")  # adam.ts:93
        super().__init__(params, o)

    def step(self):
        """One update (adam.ts:96-120).  With capturable=True every
        parameter's step count lives in device memory and the step can be
        captured in a hip.Graph (take one step eagerly first: the moments
        and the count are created then)."""
        if capturing() and not all(g.get("capturable") for g in self.param_groups):
            # the bias corrections use the step count, a host value that a
            # replay would repeat
            raise RuntimeError("Adam / AdamW steps are captured in a graph only with "
                               "capturable=True")
        lib = L.lib()
        # the step writes parameters (and their moments) in place: deferred
        # values that read them are evaluated first
        _before_write(*[p for g in self.param_groups for p in g["params"]])
        for g in self.param_groups:
            b1, b2 = g["betas"]
            ps, gs, ms, vs, ns, steps = [], [], [], [], [], []
            for p in g["params"]:
                if p.grad is None:
                    continue
                st = self.state.get(id(p))
                if st is None:
                    if capturing():
                        raise RuntimeError("take one Adam step before capturing it in a graph")
                    st = {"step": 0, "exp_avg": zeros(p.shape), "exp_avg_sq": zeros(p.shape),
                          "param": p}
                    if g.get("capturable"):
                        st["step_dev"] = zeros((2,), dtype="int32")  # one int64 counter
                    self.state[id(p)] = st
                st["step"] += 1
                if not p.is_contiguous():
                    raise RuntimeError("Adam: parameters must be contiguous")
                grad = p.grad if p.grad.is_contiguous() else _k_contiguous(p.grad)
                p.grad = grad
                ps.append(p.data_ptr())
                gs.append(grad.data_ptr())
                ms.append(st["exp_avg"].data_ptr())
                vs.append(st["exp_avg_sq"].data_ptr())
                ns.append(p.numel())
                steps.append(st["step_dev"].data_ptr() if g.get("capturable") else st["step"])
            if not ps:
                continue
            n = len(ps)
            arr = lambda xs: (ctypes.c_void_p * n)(*xs)
            if g.get("capturable"):
                L.check(lib.tjh_adam_step_dev(n, arr(ps), arr(gs), arr(ms), arr(vs),
                                              (ctypes.c_int64 * n)(*ns), arr(steps),
                                              float(g["lr"]), float(b1), float(b2),
                                              float(g["eps"]), float(g["weight_decay"]),
                                              self._decoupled), "adam_step")
                continue
            L.check(lib.tjh_adam_step(n, arr(ps), arr(gs), arr(ms), arr(vs),
                                      (ctypes.c_int64 * n)(*ns), (ctypes.c_int64 * n)(*steps),
                                      float(g["lr"]), float(b1), float(b2), float(g["eps"]),
                                      float(g["weight_decay"]), self._decoupled), "adam_step")
        return None


class AdamW(Adam):
    """AdamW (src/optim/adamw.ts:46-154): decoupled decay p *= 1 - lr*wd,
    default weight_decay 1e-2 (adamw.ts:33-37)."""

    _decoupled = 1
    _default_wd = 1e-2


class SGD(Optimizer):
    """Plain SGD: p -= lr * (g + wd * p)."""

    def __init__(self, params, options=None, **kwargs):
        o = _opts(options, kwargs, {"lr": 1e-2, "momentum": 0.0, "weight_decay": 0.0})
        if o["momentum"]:
            raise NotImplementedError("SGD momentum is not on the hip path")
        super().__init__(params, o)

    def step(self):
        lib = L.lib()
        # parameters (and, with weight decay, gradients) are written in place
        ps = [p for g in self.param_groups for p in g["params"]]
        _before_write(*ps, *[p.grad for p in ps if p.grad is not None])
        for g in self.param_groups:
            for p in g["params"]:
                if p.grad is None:
                    continue
                grad = p.grad if p.grad.is_contiguous() else _k_contiguous(p.grad)
                if g["weight_decay"]:
                    L.check(lib.tjh_axpy(float(g["weight_decay"]), p.data_ptr(), grad.data_ptr(),
                                         grad.data_ptr(), p.numel()), "sgd")
                L.check(lib.tjh_axpy(-float(g["lr"]), grad.data_ptr(), p.data_ptr(),
                                     p.data_ptr(), p.numel()), "sgd")
        return None
