"""A float Wan block as a torch module with the reference WanBlock's structure and names (models/block.py:11-29,
multi_head_attention.py:8-44, layer_norm.py, rms_norm.py), for the conversion tests (the reference itself is not
importable where the tests run). Weights from an oracle.block.random_block dict."""

import torch

from oracle import rope as orope


class RMSNorm(torch.nn.Module):
    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.eps, self.weight = eps, torch.nn.Parameter(torch.ones(dim))

    def forward(self, x):
        x32 = x.float()
        return (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.eps)).type_as(x) * self.weight


class Attention(torch.nn.Module):
    def __init__(self, dim, heads):
        super().__init__()
        self.dim, self.num_heads, self.head_dim = dim, heads, dim // heads
        self.q, self.k, self.v, self.o = (torch.nn.Linear(dim, dim) for _ in range(4))
        self.norm_q, self.norm_k = RMSNorm(dim), RMSNorm(dim)

    def forward(self, X, grid_sizes=None, freq=None, context=None, start_frame=0, cache=None, context_kv=None):
        B, L = X.shape[0], X.shape[-2]
        shape = lambda t: t.reshape(B, -1, self.num_heads, self.head_dim)
        Q = shape(self.norm_q(self.q(X)))
        if context is not None:
            K, V = shape(self.norm_k(self.k(context))), shape(self.v(context))
        else:
            K, V = shape(self.norm_k(self.k(X))), shape(self.v(X))
            g = grid_sizes[0]
            Q = orope.rope_apply(Q.float(), g, freq.double(), start_frame).type_as(X)
            K = orope.rope_apply(K.float(), g, freq.double(), start_frame).type_as(X)
        A = torch.nn.functional.scaled_dot_product_attention(Q.transpose(1, 2).float(), K.transpose(1, 2).float(),
                                                             V.transpose(1, 2).float())
        return self.o(A.transpose(1, 2).reshape(B, L, self.dim).type_as(X))


class FloatWanBlock(torch.nn.Module):
    def __init__(self, dim, ffn, heads, eps=1e-6):
        super().__init__()
        self.self_attn, self.cross_attn = Attention(dim, heads), Attention(dim, heads)
        self.ffn = torch.nn.Sequential(torch.nn.Linear(dim, ffn), torch.nn.GELU(approximate="tanh"),
                                       torch.nn.Linear(ffn, dim))
        self.norm1 = torch.nn.LayerNorm(dim, eps=eps, elementwise_affine=False)
        self.norm3 = torch.nn.LayerNorm(dim, eps=eps, elementwise_affine=True)
        self.norm2 = torch.nn.LayerNorm(dim, eps=eps, elementwise_affine=False)
        self.modulation = torch.nn.Parameter(torch.randn(1, 6, dim) / dim ** 0.5)

    def forward(self, X, time_in, grid_sizes=None, freqs=None, context=None, start_frame=0, cache=None):
        ln = lambda m, x: m(x.float()).type_as(x)
        sh_a, sc_a, g_a, sh_f, sc_f, g_f = (time_in + self.modulation).chunk(6, dim=1)
        X = X + self.self_attn(ln(self.norm1, X) * (1 + sc_a) + sh_a, grid_sizes=grid_sizes, freq=freqs,
                               start_frame=start_frame, cache=cache) * g_a
        X = X + self.cross_attn(ln(self.norm3, X), context=context)
        return X + self.ffn(ln(self.norm2, X) * (1 + sc_f) + sh_f) * g_f

    @classmethod
    def from_random_block(cls, B, dim, ffn, heads):
        blk = cls(dim, ffn, heads)
        W = B["W"]
        with torch.no_grad():
            for (mod, names) in ((blk.self_attn, ("q", "k", "v", "o")), (blk.cross_attn, ("cq", "ck", "cv", "co"))):
                for attr, n in zip(("q", "k", "v", "o"), names):
                    getattr(mod, attr).weight.copy_(W[n][0])
                    getattr(mod, attr).bias.copy_(W[n][1])
            blk.self_attn.norm_q.weight.copy_(B["wq"])
            blk.self_attn.norm_k.weight.copy_(B["wk"])
            blk.cross_attn.norm_q.weight.copy_(B["cwq"])
            blk.cross_attn.norm_k.weight.copy_(B["cwk"])
            blk.ffn[0].weight.copy_(W["ffn1"][0]), blk.ffn[0].bias.copy_(W["ffn1"][1])
            blk.ffn[2].weight.copy_(W["ffn2"][0]), blk.ffn[2].bias.copy_(W["ffn2"][1])
            blk.norm3.weight.copy_(B["n3w"]), blk.norm3.bias.copy_(B["n3b"])
            blk.modulation.copy_(B["modulation"].reshape(1, 6, dim))
        return blk
