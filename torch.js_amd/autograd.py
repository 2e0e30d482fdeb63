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
    inputs, without touching .grad.  With create_graph the gradients carry
    graphs of their own, so grad() can be applied to them again (second
    derivatives); retain_graph then defaults to True, as in PyTorch."""
    single = isinstance(inputs, Tensor)
    inputs = [inputs] if single else list(inputs)
    if retain_graph is None:
        retain_graph = create_graph
    res = run_backward(_pairs(outputs, grad_outputs), retain_graph=bool(retain_graph),
                       inputs=inputs, create_graph=bool(create_graph))
    for t, r in zip(inputs, res):
        if r is None and not allow_unused:
            raise RuntimeError("One of the differentiated Tensors appears to not have been used "
                               "in the graph. Set allow_unused=True if this is the desired behavior.")
    return tuple(res)


def backward(tensors, grad_tensors=None, retain_graph=None, create_graph=False):
    if retain_graph is None:
        retain_graph = create_graph
    run_backward(_pairs(tensors, grad_tensors), retain_graph=retain_graph,
                 create_graph=create_graph)


def vjp(func, inputs, v=None, create_graph=False):
    """autograd.functional.vjp (src/autograd.ts:74-86): (func(inputs), v^T J).
    With create_graph the product carries a graph back to `inputs` (which
    keep requiring grad), so it can be differentiated again."""
    single = isinstance(inputs, Tensor)
    ins = [inputs] if single else list(inputs)
    if not create_graph:
        ins = [i.detach().requires_grad_(True) for i in ins]
    out = func(*ins)
    g = grad(out, ins, grad_outputs=v, allow_unused=True, create_graph=create_graph)
    return (out if create_graph else out.detach()), (g[0] if single else g)


def jvp(func, inputs, v, create_graph=False):
    """autograd.functional.jvp (src/autograd.ts:88-137): (func(x), J v) for
    one input tensor, by reverse mode as torch.js computes it: element i of
    J v is <d out_i / dx, v>, one retained backward pass per output element
    (a scalar output takes one).  The dot products and the result stay on
    the device (torch.js reads each one back)."""
    from .tensor import _k_reduce, _k_binary, _view_raw, cat, reshape_raw, zeros
    if not isinstance(inputs, Tensor):
        raise TypeError("jvp: one input tensor is supported")
    x = inputs.detach().requires_grad_(True)
    out = func(x)
    vf = reshape_raw(v.contiguous(), (v.numel(),))
    n = out.numel()
    parts = []
    for i in range(n):
        e = zeros(out.shape)
        if n > 1:
            _view_raw(e, (n,))[i].fill_(1.0)
        else:
            e.fill_(1.0)
        (gi,) = grad(out, x, grad_outputs=e, retain_graph=True, allow_unused=True)
        if gi is None:
            parts.append(zeros((1,)))
            continue
        prod = _k_binary("mul", reshape_raw(gi.contiguous(), (gi.numel(),)), vf)
        parts.append(_view_raw(_k_reduce("sum", prod, [0]), (1,)))
    res = cat(parts, 0) if parts else zeros((0,))
    return out.detach(), reshape_raw(res, out.shape)


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
            # with create_graph the engine runs backward() in grad mode, so
            # the user's ops record the gradient's own graph (gfn = fn)
            out.grad_fn = Node(cls.__name__, [t if t.requires_grad else None for t in tens], fn,
                               gfn=fn)
        return out

    @staticmethod
    def forward(ctx, *args):
        raise NotImplementedError

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError
