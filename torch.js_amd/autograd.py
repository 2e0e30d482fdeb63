"""torch.autograd for the 'hip' device (src/autograd.ts:22-204):
grad / backward / vjp and custom Functions over the tensor engine."""
from .tensor import (Node, Tensor, _grad, full, is_grad_enabled, no_grad, run_backward)


def _pairs(outputs, grad_outputs):
    if isinstance(outputs, Tensor):
        outputs = [outputs]
    outputs = list(outputs)
    if grad_outputs is None:
        grad_outputs = [None] * len(outputs)
    elif isinstance(grad_outputs, Tensor):
        grad_outputs = [grad_outputs]
    pairs = []
    for o, g in zip(outputs, grad_outputs):
        if g is None:
            if o.numel() != 1:
                raise RuntimeError("grad can be implicitly created only for scalar outputs")
            g = full(o.shape, 1.0)
        pairs.append((o, g))
    return pairs


def grad(outputs, inputs, grad_outputs=None, retain_graph=None, create_graph=False,
         allow_unused=False):
    """autograd.grad (src/autograd.ts:22-72): gradients of outputs w.r.t.
    inputs, without touching .grad."""
    if create_graph:
        raise NotImplementedError("create_graph=True is not supported on the hip device")
    single = isinstance(inputs, Tensor)
    inputs = [inputs] if single else list(inputs)
    res = run_backward(_pairs(outputs, grad_outputs), retain_graph=bool(retain_graph),
                       inputs=inputs)
    for t, r in zip(inputs, res):
        if r is None and not allow_unused:
            raise RuntimeError("One of the differentiated Tensors appears to not have been used "
                               "in the graph. Set allow_unused=True if this is the desired behavior.")
    return tuple(res)


def backward(tensors, grad_tensors=None, retain_graph=False):
    run_backward(_pairs(tensors, grad_tensors), retain_graph=retain_graph)


def vjp(func, inputs, v=None):
    """autograd.functional.vjp (src/autograd.ts:74-105): (func(inputs), v^T J)."""
    single = isinstance(inputs, Tensor)
    ins = [inputs] if single else list(inputs)
    ins = [i.detach().requires_grad_(True) for i in ins]
    out = func(*ins)
    g = grad(out, ins, grad_outputs=v, allow_unused=True)
    return out.detach(), (g[0] if single else g)


class _Ctx:
    def __init__(self):
        self.saved_tensors = ()
        self.needs_input_grad = ()

    def save_for_backward(self, *tensors):
        self.saved_tensors = tuple(tensors)


class Function:
    """Custom autograd function (src/autograd.ts:145-182): subclass with
    static forward(ctx, *args) and backward(ctx, *grads); call apply()."""

    @classmethod
    def apply(cls, *args):
        ctx = _Ctx()
        tens = [a for a in args if isinstance(a, Tensor)]
        ctx.needs_input_grad = tuple(isinstance(a, Tensor) and a.requires_grad for a in args)
        with no_grad():
            out = cls.forward(ctx, *args)
        if not isinstance(out, Tensor):
            raise TypeError("Function.forward must return a single Tensor")
        if is_grad_enabled() and any(t.requires_grad for t in tens):
            positions = [i for i, a in enumerate(args) if isinstance(a, Tensor)]

            def fn(g):
                gs = cls.backward(ctx, g)
                if not isinstance(gs, (tuple, list)):
                    gs = (gs,)
                return [gs[i] if i < len(gs) else None for i in positions]
            out = out.detach()
            out.requires_grad = True
            out.grad_fn = Node(cls.__name__, [t if t.requires_grad else None for t in tens], fn)
        return out

    @staticmethod
    def forward(ctx, *args):
        raise NotImplementedError

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError
