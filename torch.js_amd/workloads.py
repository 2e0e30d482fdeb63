"""The benchmark workloads as torch.js programs on the 'hip' device.

Each is written against this package's public API exactly as a torch.js
user would write it (nn modules, functional ops, backward(), optimizers):
  * MLP     Linear(784,256) -> ReLU -> Linear(256,10), cross_entropy, Adam
  * chain   (x + bias) -> GELU -> * y -> sum(0) -> mean
  * CNN     conv 3->32 3x3 p1 -> ReLU -> conv 32->64 3x3 s2 p1 -> ReLU ->
            global avg-pool -> Linear(64,10) -> cross_entropy
  * Block   pre-LN transformer block (causal SDPA, 4x GELU MLP)
  * GPT2    GPT-2 small with tied embeddings, next-token cross_entropy
"""
from . import functional as F
from . import nn
from .tensor import arange, from_numpy


def mlp():
    return nn.Sequential(nn.Linear(784, 256), nn.ReLU(), nn.Linear(256, 10))


def chain_loss(x, bias, y):
    return (F.gelu(x + bias) * y).sum(0).mean()


class CNN(nn.Module):
    def __init__(self):
        super().__init__()
        self.conv1 = nn.Conv2d(3, 32, 3, padding=1)
        self.conv2 = nn.Conv2d(32, 64, 3, stride=2, padding=1)
        self.fc = nn.Linear(64, 10)

    def forward(self, x):
        x = F.relu(self.conv1(x))
        x = F.relu(self.conv2(x))
        return self.fc(x.mean((2, 3)))


class CausalSelfAttention(nn.Module):
    def __init__(self, d, heads, fused=True):
        super().__init__()
        self.d, self.heads, self.fused = d, heads, fused
        self.c_attn = nn.Linear(d, 3 * d)
        self.c_proj = nn.Linear(d, d)

    def forward(self, x, residual=None):
        """attention(x), or residual + attention(x) (with `fused`, the add is
        done by the output projection's GEMM epilogue; without, it is the
        public `+`)."""
        B, T, C = x.shape
        hd = C // self.heads
        q, k, v = self.c_attn(x).split(C, dim=2)
        q = q.view(B, T, self.heads, hd).transpose(1, 2)
        k = k.view(B, T, self.heads, hd).transpose(1, 2)
        v = v.view(B, T, self.heads, hd).transpose(1, 2)
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        y = y.transpose(1, 2).contiguous().view(B, T, C)
        if self.fused:
            return F._linear_add(y, self.c_proj.weight, self.c_proj.bias, residual)
        out = self.c_proj(y)
        return out if residual is None else residual + out


class MLPBlock(nn.Module):
    def __init__(self, d, fused=True):
        super().__init__()
        self.fused = fused
        self.c_fc = nn.Linear(d, 4 * d)
        self.c_proj = nn.Linear(4 * d, d)

    def forward(self, x, residual=None):
        if self.fused:
            # c_proj(gelu(c_fc(x))) (+ residual) with GELU and the add fused
            # into the two GEMMs
            return F._mlp_gelu(x, self.c_fc.weight, self.c_fc.bias, self.c_proj.weight,
                               self.c_proj.bias, residual)
        out = self.c_proj(F.gelu(self.c_fc(x)))
        return out if residual is None else residual + out


class Block(nn.Module):
    """Pre-LayerNorm transformer block.  fused=False writes it with the
    public operators only (nn.Linear, F.gelu, `+`), as a torch.js program
    would; fused=True routes the GELU and the residual adds through the
    GEMM epilogues (the same values, bit for bit)."""

    def __init__(self, d, heads, fused=True):
        super().__init__()
        self.ln_1 = nn.LayerNorm(d)
        self.attn = CausalSelfAttention(d, heads, fused)
        self.ln_2 = nn.LayerNorm(d)
        self.mlp = MLPBlock(d, fused)

    def forward(self, x):
        # x + attn(ln_1(x)), then x + mlp(ln_2(x))
        x = self.attn(self.ln_1(x), residual=x)
        return self.mlp(self.ln_2(x), residual=x)


class GPT2(nn.Module):
    """GPT-2 with the LM head tied to the token embedding."""

    def __init__(self, vocab=50257, ctx=1024, d=768, heads=12, layers=12, fused=True):
        super().__init__()
        self.vocab, self.ctx = vocab, ctx
        self.wte = nn.Embedding(vocab, d)
        self.wpe = nn.Embedding(ctx, d)
        self.h = nn.ModuleList([Block(d, heads, fused) for _ in range(layers)])
        self.ln_f = nn.LayerNorm(d)

    def forward(self, ids):
        B, T = ids.shape
        pos = arange(T, dtype="int32")
        x = self.wte(ids) + self.wpe(pos)
        for blk in self.h:
            x = blk(x)
        x = self.ln_f(x)
        return F.linear(x, self.wte.weight)

    def loss(self, ids, targets):
        logits = self(ids)
        return F.cross_entropy(logits.view(-1, self.vocab), targets.reshape(-1))


def load_params(model, params):
    """Copies a {name: float32 array} dict into the model's parameters."""
    model.load_state_dict({k: from_numpy(v) for k, v in params.items()
                           if k in dict(model.named_parameters())})
    return model
