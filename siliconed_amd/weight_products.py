"""The model-facing product over a map: `WeightProducts.linear(name, a, c, m, k, n)` — the reference's
operator (`WeightProducts.linear(_:a:c:m:k:n:target:rounded:)`, Sources/Siliconed/WeightProducts.swift:278-436)
reduced to what reaches this library: the named tensor's route chosen as its `prepare` chooses it
(:874-959, with `readableInt8` :801-807 and `quantizedPlan` :864-872), the weight staged once
(`Artifact.stageInt8`'s place, Artifact.swift:755-774: the packed layout, kept on the device per name
instead of copied into a reserve per product), then the product on `TensorGEMM`.

Routes, in `prepare`'s order:
  * a published 8-bit weight `[k, n]` (int8; float8_e4m3 too, which the reference widens and this
    library multiplies natively) with a scale for the tensor or per column, or int8 with block scales
    `[k/b, n]` (GGUF Q8_0): the 8-bit product — W8A8 when the caller quantizes its activations and the
    weight is int8 per column or tensor (quantizedPlan), else on the activation rounded to bf16 when the
    caller rounds its activations (the reference's `roundsActivations`), else on the fp32 activation
    used whole (the fp32 route); a convrot weight's rotation (`Artifact.Rotation`) goes to the activation;
  * a bf16 weight `[k, n]`: the bf16-weight product, on the rounded or the fp32 activation likewise;
  * anything else — an SQ or packed code, an fp32 or fp16 weight, a shape other than `[k, n]` — is
    the reference's widened route (`widen`, `GEMM.linear`), which this library does not hold:
    `abi.Unsupported`, raised before any work, as the caller's signal to widen.
The reference's other partners of the product (the ANE's rows, the AMX's columns, LoRA, the ledger)
are not this library's; the route for a tensor is `route(name, k, n)`, the product `linear`.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import torch

from . import _abi as abi
from .artifact import Artifact, ArtifactError, StagedWeight


@dataclass(frozen=True)
class Route:
    """How `linear` multiplies a tensor: `weight` (int8, float8_e4m3, q8_0 or bfloat16), `activation`
    ("rounded" to bf16, "fp32" used whole, or "quantized" per row: W8A8), the convrot `group` (0: none)
    and the block size of block scales (None: per column or tensor)."""
    weight: str
    activation: str
    group: int = 0
    block: Optional[int] = None


class WeightProducts:
    """`WeightProducts` over one map (an `Artifact`) and one `TensorGEMM` context.

    `rounds_activations` / `quantizes_activations`: the caller's `roundsActivations` and W8A8 choice
    (the reference's plan asks per product; here one choice per operator). Staged weights stay on the
    device until `release`."""

    def __init__(self, artifact: Artifact, gemm=None, *, rounds_activations: bool = True,
                 quantizes_activations: bool = False, device: int = 0):
        from .tensor_gemm import context
        self.artifact = artifact
        self.gemm = gemm or context(device)
        self.rounds_activations = rounds_activations
        self.quantizes_activations = quantizes_activations
        self.device = torch.device("cuda", device)
        self._staged: Dict[tuple, object] = {}

    # ---- the route (prepare) --------------------------------------------------------------------

    def route(self, name: str, k: int, n: int) -> Route:
        """`prepare`'s choice for `name` as a [k, n] product; `abi.Unsupported` where the reference
        widens; ArtifactError where its count disagrees with k·n (`expect`, WeightProducts.swift:875-877)."""
        t = self.artifact.tensors.get(name)
        if t is None:
            raise ArtifactError("missing", f"{name}: no such tensor in the map", self.artifact.path)
        if t.count != k * n:
            raise ArtifactError("bad_header", f"{name}: {t.count} values, {k * n} expected", self.artifact.path)
        if t.shape != [k, n]:
            raise abi.Unsupported(abi.EUNSUPPORTED, f"{name}: shape {t.shape} is not [{k}, {n}] (the widened route)")
        activation = "rounded" if self.rounds_activations else "fp32"
        if t.dtype == "bfloat16":
            return Route("bfloat16", activation)
        if t.dtype not in ("int8", "float8_e4m3") or t.scale is None:
            raise abi.Unsupported(abi.EUNSUPPORTED, f"{name}: {t.dtype} is not an 8-bit weight of this library "
                                                    "(the widened route)")
        group = t.rotation.group if t.rotation else 0
        if t.scale.layout == "blocks":
            if t.dtype != "int8" or group:
                raise abi.Unsupported(abi.EUNSUPPORTED, f"{name}: block scales take int8 codes and no rotation")
            return Route("q8_0", activation, 0, t.scale.block)
        if self.quantizes_activations and t.dtype == "int8":
            return Route("int8", "quantized", group)
        return Route(t.dtype, activation, group)

    # ---- staging ------------------------------------------------------------------------------------

    def staged(self, name: str, glu: bool = False):
        """The weight on the device, staged once: a StagedWeight (8-bit codes packed, fp32 scale or
        block scales), or the bf16 weight [k, n] itself."""
        key = (name, glu)
        w = self._staged.get(key)
        if w is None:
            t = self.artifact.tensors[name]
            if t.dtype == "bfloat16":
                bits = torch.from_numpy(self.artifact.values(name).copy().view("int16"))
                w = bits.view(torch.bfloat16).to(self.device)
            else:
                w = self.artifact.stage(name, self.gemm, device=self.device.index or 0, glu=glu)
            self._staged[key] = w
        return w

    def release(self, name: Optional[str] = None) -> None:
        """Frees the staged copy of `name` (all names: None)."""
        for key in [key for key in self._staged if name is None or key[0] == name]:
            del self._staged[key]

    # ---- the product --------------------------------------------------------------------------------

    def linear(self, name: str, a: torch.Tensor, c: torch.Tensor, m: int, k: int, n: int, *,
               bias: Optional[torch.Tensor] = None, epilogue=None) -> float:
        """C fp32 [m, n] (written; [m, n/2] for a GLU epilogue) = A [m, k] · W, W the map's `name` [k, n]
        by `route` — A fp32, or bf16 when its producer rounded it already (the reference's `rounded`
        operand). `bias` / `epilogue`: fused after the scale (this library's; the reference's callers
        run them as passes). Returns the GPU seconds."""
        r = self.route(name, k, n)
        glu = epilogue in ("silu_glu", "situ_glu")
        n_out = n // 2 if glu else n
        if a.numel() < m * k or c.numel() < m * n_out or c.dtype != torch.float32:
            raise ValueError("a smaller than m × k, or c not fp32 with m × n values")
        x = a.reshape(-1)[: m * k].view(m, k)
        out = c.reshape(-1)[: m * n_out].view(m, n_out)
        g = self.gemm
        # The products run on the caller's current stream, ordered with its other work (the context
        # waits for its previous stream's work when the stream changes).
        g.set_stream(torch.cuda.current_stream(self.device))
        if r.weight == "bfloat16":
            if epilogue is not None or bias is not None:
                raise abi.Unsupported(abi.EUNSUPPORTED, f"{name}: the bf16-weight product takes no bias or epilogue")
            w = self.staged(name)
            if r.activation == "rounded" and x.dtype == torch.float32:
                x = g.round_bf16(x)
            _, secs = g.product_bf16_weight(x, w, layout="kn", out=out, timed=True)
            return secs
        w = self.staged(name, glu=glu)
        assert isinstance(w, StagedWeight)
        if r.activation == "quantized":
            _, secs = g.product_quantized(x, w.packed, w.scale, group=r.group, bias=bias, epilogue=epilogue, out=out,
                                          out_dtype=torch.float32, timed=True)
        elif r.block is not None:
            _, secs = g.product_blocks(x, w.packed, bias=bias, epilogue=epilogue, out=out, out_dtype=torch.float32,
                                       timed=True, rounding=r.activation == "rounded")
        else:
            _, secs = g.product(x, w.packed, w.scale, bias=bias, epilogue=epilogue, out=out, out_dtype=torch.float32,
                                timed=True, rotation=r.group, rounding=r.activation == "rounded")
        return secs
