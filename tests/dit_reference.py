"""The checker of the synthetic DiT block (siliconed_amd.dit_block): the same block in fp32 with the
dequantised weights Float(q)·s and fp32 math attention, its operands rounded to bf16 where the block
rounds them — or, on the W8A8 route, rotated and quantized per row as the block quantizes them (the
product of a rotated operand with the stored weight is the product with the convrot weight (q·s)·R).
Test infrastructure: the product path never imports it."""
from __future__ import annotations

import torch

from siliconed_amd.dit_block import EPS


def rms_modulate(x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                 to_bf16: bool = True) -> torch.Tensor:
    """RMS(x)·w·(1 + scale) + shift, fp32 arithmetic; rounded to bf16 (the next product's operand on
    the bf16 route) unless `to_bf16` is false (the W8A8 route quantizes the fp32 row)."""
    r = torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + EPS)
    y = (x * r) * w * (1.0 + scale) + shift
    return y.to(torch.bfloat16) if to_bf16 else y


def rms_heads(t: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Per-head RMSNorm of q or k, [heads, S, head_dim] bf16, fp32 arithmetic."""
    t32 = t.float()
    return (t32 * torch.rsqrt(t32.pow(2).mean(dim=-1, keepdim=True) + EPS) * w).to(torch.bfloat16)


def rotate(a: torch.Tensor, g: int) -> torch.Tensor:
    """a·R by groups of g in fp32 (R = H/√g, H the Kronecker power of the regular H4); g = 0: a."""
    if not g:
        return a
    h4 = torch.tensor([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=torch.float32, device=a.device)
    h = torch.ones((1, 1), device=a.device)
    while h.shape[0] < g:
        h = torch.kron(h, h4)
    return (a.reshape(a.shape[0], -1, g) @ (h / g ** 0.5)).reshape(a.shape)


def quantized(a: torch.Tensor, g: int) -> torch.Tensor:
    """The W8A8 operand in fp32: a rotated, quantized per row (s = max|y|/127, rint) and scaled back."""
    y = rotate(a.float(), g)
    s = (y.abs().amax(dim=1, keepdim=True) / 127.0).clamp_min(1e-30)
    return torch.round(y / s).clamp(-128, 127) * s


def reference(blk, x: torch.Tensor, temb: torch.Tensor, rows=None) -> torch.Tensor:
    """The block's output in fp32 for x fp32 [S, d] and temb [d]; with `rows` (a LongTensor) only those
    rows of the output (the attention still sees every key and value; the row-wise parts after it run
    on the sampled rows alone)."""
    w8 = blk.route == "w8a8"

    def lin(a, L, act=None, quant=None):
        quant = w8 if quant is None else quant
        a = quantized(a, blk.group) if quant else a.float()
        y = a @ (L["q"].float() * L["s"][:, None]).t() + L["b"]
        return torch.nn.functional.gelu(y, approximate="tanh") if act else y

    S, d = x.shape
    mod = lin(temb.to(torch.bfloat16)[None], blk.mod, quant=False)[0]
    shift_a, scale_a, gate_a, shift_f, scale_f, gate_f = mod.chunk(6)
    n = rms_modulate(x, blk.norm_a, scale_a, shift_a, to_bf16=not w8)
    qkv = lin(n, blk.qkv).to(torch.bfloat16).view(S, 3, blk.heads, blk.hd).permute(1, 2, 0, 3)
    q, k, v = (rms_heads(t.contiguous(), w).float() if w is not None else t.float()
               for t, w in zip(qkv, (blk.norm_q, blk.norm_k, None)))
    if rows is not None:
        q, x = q[:, rows], x[rows]
    att = torch.softmax((q @ k.transpose(1, 2).contiguous()) / blk.hd ** 0.5, dim=-1) @ v
    o = att.to(torch.bfloat16).transpose(0, 1).reshape(x.shape[0], d)
    x = x + gate_a * lin(o, blk.out)
    m = rms_modulate(x, blk.norm_f, scale_f, shift_f, to_bf16=not w8)
    h = lin(m, blk.up, act=True).to(torch.bfloat16)
    return x + gate_f * lin(h, blk.down)
