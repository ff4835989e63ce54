"""bench.CpuBlock (the CPU baseline's PyTorch block) against the oracle's quantized block on the same weights: the
baseline times the block this build computes, not another one.

At dim 256 (2 heads, FFN 512, 2 x 4 x 6 tokens over a 96-token FP8 cache and a 16-token prompt), fp32: the
block's update (out - X) within 12 % relative L2 of the oracle's (oracle.block.block_forward). The two differ in the
last bits everywhere (torch's LayerNorm order, fp32 where the oracle rounds to bf16, exact SDPA on the dequantized
cache where the oracle runs Sage attention), and a W4A4 block with these random weights is chaotic at that level:
the oracle's own update moves by 4.9 % when 20 of its 12 288 input entries move by one bf16 step. Measured 8.4 %.
Swapping the attention and feed-forward gates in CpuBlock's modulation moves it by 0.30, more than twice the bar."""

import torch

import bench
from oracle import block as oblock
from oracle import rope as orope


def _case(blk, g):
    dim, heads, grid, prior, Lc = blk.dim, blk.heads, (2, 4, 6), 96, 16
    M = grid[0] * grid[1] * grid[2]
    X = torch.randn(M, dim, generator=g).to(torch.bfloat16)
    time_in = torch.randn(6, dim, generator=g) * 0.1
    C = torch.randn(Lc, dim, generator=g).to(torch.bfloat16)
    ck = (torch.randn(1, prior + M, heads, 128, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    cs = torch.rand(1, prior + M, heads, 1, generator=g) * 0.02
    P = blk.oracle_parts()
    Kc, Vc = oblock.context_kv(C, P)
    ref = oblock.block_forward(X, time_in, P, grid, orope.freqs(128, 1024, torch.float64).float(), 3,
                               dict(k=ck.clone(), ks=cs.clone(), v=ck.clone(), vs=cs.clone(), at=prior), (Kc, Vc),
                               heads)
    cache = (ck[0, :prior].float() * cs[0, :prior]).float()
    args = (X.float(), time_in, cache, cache, Kc.float().view(Lc, heads, 128), Vc.float().view(Lc, heads, 128),
            grid, 3)
    return X, ref, args


def test_cpu_block_is_the_oracle_block():
    g = torch.Generator().manual_seed(3)
    blk = bench.CpuBlock(torch.float32, seed=5, dim=256, ffn=512, heads=2)
    X, ref, args = _case(blk, g)
    with torch.no_grad():
        out = blk.forward(*args)
    du, dr = out.float() - X.float(), ref.float() - X.float()
    err = float((du - dr).norm() / dr.norm())
    print(f"CpuBlock vs oracle block: update rel-L2 {err:.3e}")
    assert err <= 0.12
    blk.mod = blk.mod[[0, 1, 5, 3, 4, 2]]  # the gates swapped: a wiring mistake the bar must catch
    with torch.no_grad():
        bad = blk.forward(*args)
    planted = float(((bad.float() - X.float()) - dr).norm() / dr.norm())
    print(f"with the gates swapped: {planted:.3f}")
    assert planted > 2 * 0.12  # the wiring mistake fails the bar by a wide margin
