"""A synthetic single-stream DiT block on the weight-quantized linear layer: the C4 workload.

One block of MossImage.swift:15-19 with the 4× GELU-tanh MLP of the other DiT targets:

    n = RMS(x)·w_a·(1 + scale_a) + shift_a
    x += gate_a · Wo( SDPA(RMS_h(Wq n), RMS_h(Wk n), Wv n) )        (heads of 128, no mask)
    m = RMS(x)·w_f·(1 + scale_f) + shift_f
    x += gate_f · W_down( GELU_tanh(W_up m) )

with the six modulation vectors [shift_a, scale_a, gate_a, shift_f, scale_f, gate_f] from one Linear
of the timestep embedding (MossImage.swift:23-27: no SiLU before it, the shift first, plain gates).

`route="w8a8"`: the block's products on the W8A8 route (ComfyUI's int8_linear,
TensorGEMMInt8.swift:4-37) with convrot weights of rotation group `group` (0: none): the norms write
the QKV and W_up operands as int8 codes themselves (sq8_norm_modulate_quantized, the reference's
norm_modulate_quantized), the attention output and the GELU output are quantized by the quantization
pass, and every product but the modulation's (one row: the bf16 route's skinny kernel) is int8 × int8.
Every Linear — the modulation, the fused QKV, Wo, W_up (GELU fused) and W_down — is an int8
per-output-channel product of this library (weights w ~ N(0, 0.02), s = amax/127,
q = clamp(rint(w/s), −127, 127), staged once in the packed layout). The residual stream is fp32 as
in the reference; the products' operands are bf16. The modulated norms (eps 1e-6, MossImage.swift:49),
the per-head norms and the gated residual updates are this library's elementwise passes; the
attention is torch's fused flash / memory-efficient SDPA in bf16. RoPE is left out: an elementwise
rotation of q and k, small next to the products.
"""
from __future__ import annotations

import torch

from .tensor_gemm import TensorGEMM, context

EPS = 1e-6


def quantize_int8(w: torch.Tensor):
    """Per-output-channel int8 of an [N, K] weight: s = amax/127, q = clamp(rint(w/s), −127, 127)."""
    s = (w.abs().amax(dim=1) / 127.0).clamp_min(1e-30)
    q = torch.round(w / s[:, None]).clamp(-127, 127).to(torch.int8)
    return q, s.float()


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Softmax attention of [heads, S, head_dim] bf16, no mask, on torch's fused kernels only."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return torch.nn.functional.scaled_dot_product_attention(q[None], k[None], v[None])[0]


class DiTBlock:
    """The block's weights (int8 packed, fp32 scales, fp32 norm weights) on one device."""

    def __init__(self, d: int = 3072, heads: int = 24, mlp: int = 4, seed: int = 0, device: int = 0,
                 ctx: TensorGEMM | None = None, route: str = "bf16", group: int = 0, keep_codes: bool = False):
        """`keep_codes`: also keep each weight's int8 codes [N, K] (key "q") beside the packed copy the
        forward reads — for a checker that widens them itself; off, only the packed codes stay resident."""
        if d % heads or (d // heads) % 8:
            raise ValueError("d must split into heads of a multiple of 8")
        if route not in ("bf16", "w8a8"):
            raise ValueError("route is 'bf16' or 'w8a8'")
        self.route, self.group = route, group
        self.d, self.heads, self.hd = d, heads, d // heads
        self.ctx = ctx or context(device)
        dev = torch.device("cuda", device)
        g = torch.Generator(device=dev).manual_seed(seed)

        def linear(n_out: int, k: int):
            q, s = quantize_int8(torch.randn((n_out, k), device=dev, generator=g) * 0.02)
            b = torch.randn(n_out, device=dev, generator=g) * 0.02
            lin = {"n": n_out, "s": s, "b": b, "packed": self.ctx.pack(q, layout="nk")}
            if keep_codes:
                lin["q"] = q
            return lin

        self.mod = linear(6 * d, d)
        self.qkv = linear(3 * d, d)
        self.out = linear(d, d)
        self.up = linear(mlp * d, d)
        self.down = linear(d, mlp * d)
        self.norm_a = 1.0 + 0.02 * torch.randn(d, device=dev, generator=g)
        self.norm_f = 1.0 + 0.02 * torch.randn(d, device=dev, generator=g)
        self.norm_q = 1.0 + 0.02 * torch.randn(self.hd, device=dev, generator=g)
        self.norm_k = 1.0 + 0.02 * torch.randn(self.hd, device=dev, generator=g)

    def _product(self, x: torch.Tensor, lin: dict, epilogue=None, out_dtype=torch.bfloat16) -> torch.Tensor:
        return self.ctx.product(x, lin["packed"], lin["s"], bias=lin["b"], epilogue=epilogue, out_dtype=out_dtype)

    def _product8(self, codes_sx, lin: dict, epilogue=None, out_dtype=torch.bfloat16) -> torch.Tensor:
        codes, sx = codes_sx
        return self.ctx.product_w8a8(codes, sx, lin["packed"], lin["s"], bias=lin["b"], epilogue=epilogue,
                                     out_dtype=out_dtype)

    def _forward_w8a8(self, x: torch.Tensor, temb: torch.Tensor) -> torch.Tensor:
        S, d = x.shape
        ctx, g = self.ctx, self.group
        mod = self._product(temb.to(torch.bfloat16)[None], self.mod, out_dtype=torch.float32)[0]
        shift_a, scale_a, gate_a, shift_f, scale_f, gate_f = mod.chunk(6)
        n8 = ctx.norm_modulate_quantized(x, self.norm_a, scale_a, shift_a, EPS, g)
        q, k, v = ctx.product_w8a8_qkv(n8[0], n8[1], self.qkv["packed"], self.qkv["s"], bias=self.qkv["b"])
        ctx.rms_rows(q.view(S * self.heads, self.hd), self.norm_q, EPS)
        ctx.rms_rows(k.view(S * self.heads, self.hd), self.norm_k, EPS)
        heads = lambda t: t.view(S, self.heads, self.hd).transpose(0, 1)
        o = attention(heads(q), heads(k), heads(v)).transpose(0, 1).reshape(S, d)
        o8 = ctx.quantize_rows(o, g)
        ctx.product_w8a8_residual(x, o8[0], o8[1], self.out["packed"], self.out["s"], bias=self.out["b"], gate=gate_a)
        m8 = ctx.norm_modulate_quantized(x, self.norm_f, scale_f, shift_f, EPS, g)
        h8 = ctx.quantize_rows(self._product8(m8, self.up, epilogue="gelu_tanh"), g)
        ctx.product_w8a8_residual(x, h8[0], h8[1], self.down["packed"], self.down["s"], bias=self.down["b"], gate=gate_f)
        return x

    def forward_(self, x: torch.Tensor, temb: torch.Tensor) -> torch.Tensor:
        """The block on the residual stream x (fp32 [S, d], contiguous), updated in place as the
        reference's stream buffer is; temb [d]. Every pass but the attention is this library's: the
        modulation, the fused QKV (rows [S, heads·hd]: q, k, v are [heads, S, hd] views), Wo and W_down
        with the gated residual update fused (x += gate ⊙ product, the product in fp32), W_up with GELU
        fused; the modulated norms and the per-head norms of q and k."""
        if self.route == "w8a8":
            return self._forward_w8a8(x, temb)
        S, d = x.shape
        ctx = self.ctx
        mod = self._product(temb.to(torch.bfloat16)[None], self.mod, out_dtype=torch.float32)[0]
        shift_a, scale_a, gate_a, shift_f, scale_f, gate_f = mod.chunk(6)
        n = ctx.norm_modulate(x, self.norm_a, scale_a, shift_a, EPS)
        q, k, v = ctx.product_qkv(n, self.qkv["packed"], self.qkv["s"], bias=self.qkv["b"])   # [S, d] each
        ctx.rms_rows(q.view(S * self.heads, self.hd), self.norm_q, EPS)
        ctx.rms_rows(k.view(S * self.heads, self.hd), self.norm_k, EPS)
        heads = lambda t: t.view(S, self.heads, self.hd).transpose(0, 1)                        # [heads, S, hd]
        o = attention(heads(q), heads(k), heads(v)).transpose(0, 1).reshape(S, d)
        ctx.product_residual(x, o, self.out["packed"], self.out["s"], bias=self.out["b"], gate=gate_a)
        m = ctx.norm_modulate(x, self.norm_f, scale_f, shift_f, EPS)
        h = self._product(m, self.up, epilogue="gelu_tanh")
        ctx.product_residual(x, h, self.down["packed"], self.down["s"], bias=self.down["b"], gate=gate_f)
        return x

    def forward(self, x: torch.Tensor, temb: torch.Tensor) -> torch.Tensor:
        """x fp32 [S, d] (the residual stream), temb [d]: the block's output, fp32 [S, d] (x kept)."""
        return self.forward_(x.clone(), temb)

    def flops(self, S: int) -> float:
        """Linear FLOPs (modulation included) + attention's two products."""
        d = self.d
        lin = 2.0 * (6 * d * d + S * (3 * d * d + d * d + 2 * self.up["n"] * d))
        return lin + 4.0 * S * S * d
