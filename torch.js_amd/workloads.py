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
from .tensor import arange, from_numpy, no_grad, zeros


def mlp():
    return nn.Sequential(nn.Linear(784, 256), nn.ReLU(), nn.Linear(256, 10))


def chain_loss(x, bias, y):
    return (F.gelu(x + bias) * y).sum(0).mean()


class CNN(nn.Module):
    """conv 3->32 3x3 p1, ReLU, conv 32->64 3x3 s2 p1, ReLU, average pool,
    Linear(64, 10).  `fused`: each conv and its ReLU as one op
    (F.conv2d_relu, bit for bit the two in sequence)."""

    def __init__(self, fused=True):
        super().__init__()
        self.conv1 = nn.Conv2d(3, 32, 3, padding=1)
        self.conv2 = nn.Conv2d(32, 64, 3, stride=2, padding=1)
        self.fc = nn.Linear(64, 10)
        self.fused = fused

    def forward(self, x):
        for conv in (self.conv1, self.conv2):
            if self.fused:
                x = F.conv2d_relu(x, conv.weight, conv.bias, conv.stride, conv.padding,
                                  conv.dilation, conv.groups)
            else:
                x = F.relu(conv(x))
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
        return self._project(y, residual)

    def forward_cached(self, x, cache, layer, pos, residual=None):
        """Attention of the new positions [pos, pos + T) of x against the
        cached keys / values of positions [0, pos) plus their own; the new
        keys and values are appended to the cache.  A prompt (pos 0) is
        causal over itself; a single new token attends to every cached
        position."""
        B, T, C = x.shape
        hd = C // self.heads
        q, k, v = self.c_attn(x).split(C, dim=2)
        q = q.view(B, T, self.heads, hd).transpose(1, 2)
        k = k.view(B, T, self.heads, hd).transpose(1, 2)
        v = v.view(B, T, self.heads, hd).transpose(1, 2)
        keys, values = cache.append(layer, k, v, pos)
        if pos == 0:
            y = F.scaled_dot_product_attention(q, keys, values, is_causal=True)
        elif T == 1:
            y = F.scaled_dot_product_attention(q, keys, values, is_causal=False)
        else:
            raise NotImplementedError("KV cache: prompts start at position 0, then one token "
                                      "per step")
        y = y.transpose(1, 2).contiguous().view(B, T, C)
        return self._project(y, residual)

    def _project(self, y, residual):
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

    def forward_cached(self, x, cache, layer, pos):
        x = self.attn.forward_cached(self.ln_1(x), cache, layer, pos, residual=x)
        return self.mlp(self.ln_2(x), residual=x)


class KVCache:
    """Keys and values of every layer for positions [0, max_len): one
    [B, H, max_len, head_dim] buffer each, filled as positions arrive; the
    attention of a decoding step reads the prefix [0, pos] as a strided
    view (no copy)."""

    def __init__(self, layers, batch, heads, max_len, head_dim):
        self.max_len = max_len
        self.k = [zeros(batch, heads, max_len, head_dim) for _ in range(layers)]
        self.v = [zeros(batch, heads, max_len, head_dim) for _ in range(layers)]

    def append(self, layer, k, v, pos):
        T = k.shape[2]
        if pos + T > self.max_len:
            raise RuntimeError("KV cache: position %d beyond its length %d" % (pos + T,
                                                                              self.max_len))
        with no_grad():
            self.k[layer][:, :, pos:pos + T].copy_(k)
            self.v[layer][:, :, pos:pos + T].copy_(v)
        return self.k[layer][:, :, :pos + T], self.v[layer][:, :, :pos + T]


class GPT2(nn.Module):
    """GPT-2 with the LM head tied to the token embedding."""

    def __init__(self, vocab=50257, ctx=1024, d=768, heads=12, layers=12, fused=True):
        super().__init__()
        self.vocab, self.ctx = vocab, ctx
        self.fused = fused
        self.wte = nn.Embedding(vocab, d)
        self.wpe = nn.Embedding(ctx, d)
        self.h = nn.ModuleList([Block(d, heads, fused) for _ in range(layers)])
        self.ln_f = nn.LayerNorm(d)

    def forward(self, ids):
        x = self._embed(ids, 0)
        for blk in self.h:
            x = blk(x)
        x = self.ln_f(x)
        return F.linear(x, self.wte.weight)

    def _embed(self, ids, pos0):
        """wte(ids) + wpe(positions pos0 .. pos0 + T - 1); with `fused` one
        kernel each way (F._embedding_pos), else the public lookups and +."""
        if self.fused:
            return F._embedding_pos(ids, self.wte.weight, self.wpe.weight, pos0)
        T = ids.shape[1]
        return self.wte(ids) + self.wpe(arange(pos0, pos0 + T, dtype="int32"))

    def loss(self, ids, targets):
        logits = self(ids)
        return F.cross_entropy(logits.view(-1, self.vocab), targets.reshape(-1))

    def new_cache(self, batch, max_len=None):
        blk = self.h[0].attn
        return KVCache(len(self.h), batch, blk.heads, max_len or self.ctx, blk.d // blk.heads)

    def forward_cached(self, ids, cache, pos):
        """Logits of positions [pos, pos + T) of ids [B, T], the keys and
        values of earlier positions read from (and these appended to) the
        cache."""
        x = self._embed(ids, pos)
        for i, blk in enumerate(self.h):
            x = blk.forward_cached(x, cache, i, pos)
        x = self.ln_f(x)
        return F.linear(x, self.wte.weight)

    def generate(self, ids, max_new_tokens, temperature=1.0, greedy=False):
        """Autoregressive decoding with a KV cache (the inference side of the
        GPT-2 path, tests/gpt2.test.ts): the prompt runs once, then each
        new token is one cached step; the next token is drawn by
        multinomial from softmax(logits / temperature) (or argmax when
        greedy).  Returns the [B, T + max_new_tokens] int32 ids."""
        from .tensor import cat
        B, T = ids.shape
        total = T + max_new_tokens
        if total > self.ctx:
            raise ValueError("generate: %d positions exceed the context of %d" % (total, self.ctx))
        with no_grad():
            cache = self.new_cache(B, total)
            logits = self.forward_cached(ids, cache, 0)
            out = [ids]
            pos = T
            for _ in range(max_new_tokens):
                last = logits[:, -1, :]
                if greedy:
                    nxt = last.argmax(-1, keepdim=True)
                else:
                    probs = F.softmax(last * (1.0 / temperature), -1)
                    nxt = probs.multinomial(1)
                out.append(nxt)
                logits = self.forward_cached(nxt, cache, pos)
                pos += 1
            return cat(out, 1)


def load_params(model, params):
    """Copies a {name: float32 array} dict into the model's parameters."""
    model.load_state_dict({k: from_numpy(v) for k, v in params.items()
                           if k in dict(model.named_parameters())})
    return model
