"""The host side of the weight-quantized linear layer, over the C ABI.

`TensorGEMM` keeps the shape of the reference's operator (Sources/Siliconed/TensorGEMM.swift:59-360):
`make` is `init?` (None where the library does not run: the caller keeps its widened route),
`linear(a, int8=…, scales=…, per_column=…, c=…, m, k, n)` is `linear(a:int8:…:c:m:k:n:settled:)`
and returns the GPU seconds (0 when `settled`, i.e. queued). The memory is torch's: tensors on the
device are passed by their data pointers; torch is plumbing here, the product is the HIP library.

The functional helpers below it (`linear`, `linear_qkv`, `dequantize`, `round_bf16`) allocate their
outputs and are what the tests, the benchmark and the DiT block call.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _abi as abi

_EPILOGUES = {
    None: abi.EPI_NONE, "none": abi.EPI_NONE,
    "gelu_tanh": abi.EPI_GELU_TANH, "gelu": abi.EPI_GELU_TANH,
    "silu_glu": abi.EPI_SILU_GLU, "swiglu": abi.EPI_SILU_GLU,
    "situ_glu": abi.EPI_SITU_GLU, "situ": abi.EPI_SITU_GLU,
}
_LAYOUTS = {"kn": abi.KN, "nk": abi.NK}


class PackedWeight:
    """A weight's codes staged in the packed layout (sq8_pack_weight): `k` × `n` codes of
    `w_dtype`, paired for a GLU epilogue when `glu`. The scales stay where they were."""

    def __init__(self, data: torch.Tensor, k: int, n: int, glu: bool, w_dtype: int):
        self.data, self.k, self.n, self.glu, self.w_dtype = data, k, n, glu, w_dtype

    @property
    def layout(self) -> int:
        return abi.PACKED_GLU if self.glu else abi.PACKED


class PackedBlocks:
    """A block-scaled weight (GGUF Q8_0) staged by sq8_pack_blocks: `k` × `n` int8 codes and their
    scales per `block` rows, paired for a GLU epilogue when `glu`."""

    def __init__(self, data: torch.Tensor, k: int, n: int, glu: bool, block: int):
        self.data, self.k, self.n, self.glu, self.block = data, k, n, glu, block

    @property
    def layout(self) -> int:
        return abi.PACKED_GLU if self.glu else abi.PACKED


_SCALE_DTYPES = {torch.float32: abi.F32, torch.bfloat16: abi.BF16, torch.float16: abi.F16}


def _epilogue(name) -> int:
    if name not in _EPILOGUES:
        raise ValueError(f"unknown epilogue {name!r}")
    return _EPILOGUES[name]


def _wdtype(w: torch.Tensor, fp8: Optional[bool]) -> int:
    if w.dtype == torch.int8:
        return abi.INT8
    if w.dtype == getattr(torch, "float8_e4m3fn", None):
        return abi.FP8_E4M3
    if w.dtype == torch.uint8:
        if fp8 is None:
            raise ValueError("a uint8 weight needs fp8=True (e4m3fn codes) or an int8 view")
        return abi.FP8_E4M3 if fp8 else abi.INT8
    raise ValueError(f"weights must be int8 or float8_e4m3fn codes, not {w.dtype}")


def _adtype(a: torch.Tensor) -> int:
    if a.dtype == torch.bfloat16:
        return abi.BF16
    if a.dtype == torch.float32:
        return abi.F32
    raise ValueError(f"activations must be bfloat16 (or float32, rounded to bf16), not {a.dtype}")


def _cdtype(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return abi.BF16
    if dtype == torch.float32:
        return abi.F32
    raise ValueError(f"outputs are bfloat16 or float32, not {dtype}")


def _dev(t: torch.Tensor, what: str) -> int:
    if not t.is_cuda:
        raise ValueError(f"{what} must be on the GPU")
    return t.data_ptr()


def _row_major(t: torch.Tensor, what: str) -> int:
    """Leading dimension of a 2-D tensor whose rows are contiguous (an empty one: any strides)."""
    if t.dim() != 2 or (t.stride(1) != 1 and t.size(1) > 1 and t.size(0) > 0):
        raise ValueError(f"{what} must be 2-D with contiguous rows")
    return t.stride(0) if t.size(0) > 1 else max(t.size(1), 1)


def _block_scales(scale: Optional[torch.Tensor], lay: int, n: int, k: int, block: int, ldw: int) -> None:
    """Checks block scales against what the library reads: [n, k/block] contiguous for "nk" codes;
    for "kn" codes [k/block, n] rows with the codes' own row stride `ldw` (scale[blk·ldw + col]: a
    column-sliced weight w[:, :n] takes its scales as scale_full[:, :n])."""
    want = (n, k // block) if lay == abi.NK else (k // block, n)
    if scale is None or scale.dtype not in _SCALE_DTYPES or tuple(scale.shape) != want:
        raise ValueError(f"scale must be fp32/bf16/fp16 {want}")
    if lay == abi.NK:
        if not scale.is_contiguous():
            raise ValueError(f"scale must be contiguous {want}")
        return
    rows = want[0]
    if rows > 0 and n > 0 and ((n > 1 and scale.stride(1) != 1) or (rows > 1 and scale.stride(0) != ldw)):
        raise ValueError(f"scale {want} must have rows of stride {ldw}, the codes' row stride "
                         f"(it has strides {tuple(scale.stride())})")


class TensorGEMM:
    """One context (device + stream) of the library: `TensorGEMM` of the reference."""

    def __init__(self, handle: ctypes.c_void_p, device: int):
        self._h = handle
        self.device = device

    @classmethod
    def make(cls, device: int = 0, stream: Optional[torch.cuda.Stream] = None) -> Optional["TensorGEMM"]:
        """`init?` (TensorGEMM.swift:206-232): None when the device is not a gfx950."""
        lib = abi.load()
        h = ctypes.c_void_p()
        if stream is None and torch.cuda.is_available() and device < torch.cuda.device_count():
            stream = torch.cuda.current_stream(device)
        s = ctypes.c_void_p(stream.cuda_stream if stream is not None else None)
        st = lib.sq8_create(device, s, ctypes.byref(h))
        if st != abi.OK:
            return None
        return cls(h, device)

    def close(self) -> None:
        if self._h:
            abi.check(abi.load().sq8_destroy(self._h), "sq8_destroy")
            self._h = None

    def __del__(self):
        try:
            if self._h:
                abi.load().sq8_destroy(self._h)
                self._h = None
        except Exception:
            pass

    def set_stream(self, stream: torch.cuda.Stream) -> None:
        abi.check(abi.load().sq8_set_stream(self._h, ctypes.c_void_p(stream.cuda_stream)), "sq8_set_stream")

    def synchronize(self) -> None:
        abi.check(abi.load().sq8_synchronize(self._h), "sq8_synchronize")

    def supports(self, a_dtype: int, w_dtype: int, layout: int, scale_layout: int, c_dtype: int, epilogue: int) -> bool:
        return abi.load().sq8_supports(self._h, a_dtype, w_dtype, layout, scale_layout, c_dtype, epilogue) == abi.OK

    # ---- the reference's entry point -----------------------------------------------------------

    def linear(self, a: torch.Tensor, *, int8: torch.Tensor, scales: torch.Tensor, per_column: bool,
               c: torch.Tensor, m: int, k: int, n: int, weight_offset: int = 0, scales_offset: int = 0,
               block: Optional[int] = None, rotation=None, rounding=None, quantizing=None,
               prequantized=None, settled: bool = False, layout: str = "kn", bias: Optional[torch.Tensor] = None,
               epilogue=None, fp8: Optional[bool] = None, columns: Optional[int] = None) -> float:
        """`linear(a:int8:weightOffset:scales:scalesOffset:perColumn:…:c:m:k:n:settled:)`
        (TensorGEMM.swift:264-290): C[m, n] = A[m, k] · (q · s), q `[k, n]` (`layout="kn"`, the
        map's) at `weight_offset` bytes into `int8`, its fp32 scales at `scales_offset` bytes into
        `scales` (`n` of them, or one: `per_column` False). `a` fp32 is rounded to bf16 first when
        `rounding` is given — True or the reference's `(buffer, offset, rows)`, whose scratch this
        library replaces with its own (the `rounding:` route, TensorGEMMBF16.swift:208-264) — and
        otherwise, as the reference's default `rounding: nil`, taken whole (the fp32 route,
        sq8_linear_f32: each value split exactly into three bf16 parts, K tripled; rotated in fp32 first
        with a `rotation`; block scales too); `a` bf16 is already rounded. `rotation`: a convrot weight's group (an int, or the reference's
        `(group, scratch, offset, chunk)`, whose scratch and chunk this library replaces with its
        own), the activation rotated by it first (TensorGEMMBF16.swift:222-233). Returns the GPU
        seconds, 0 when `settled` (queued).

        `quantizing` (truthy, or the reference's `(buffer, codesOffset, scalesOffset, rows)`, whose
        reserve this library replaces with its own scratch): the W8A8 route — `a` quantized per row
        (after the rotation) and the int8 × int8 product (submitQuantized, TensorGEMMInt8.swift:237-281);
        `prequantized` = (codes, scales) of `a` already quantized skips that pass.

        Routes this library does not take raise `abi.Unsupported` before any work, as the
        reference's `nil` pipelines send the caller back to the widened route: block scales with a
        rotation or a W8A8 quantization.

        `block` = B: scales per block of B rows of K and column (GGUF Q8_0, fp32 `[k / B, n]` at
        `scales_offset`; `per_column` ignored), the product of sq8_linear_blocks.

        `columns` ≤ n: only C's first `columns` columns are computed and written (the reference's
        `submit(…columns:)`, TensorGEMM.swift:292-296); C keeps its row stride n; the weight's codes
        and block scales keep theirs. Not with a quantization or a GLU epilogue.
        """
        cols = n
        if columns is not None and columns != n:
            if not 0 <= columns <= n:
                raise ValueError(f"columns = {columns} outside [0, {n}]")
            if quantizing is not None or prequantized is not None or epilogue in ("silu_glu", "situ_glu"):
                raise abi.Unsupported(abi.EUNSUPPORTED, "columns with a quantization or a GLU epilogue")
            cols = columns
        if block is not None:
            if rotation is not None or quantizing is not None or prequantized is not None or fp8:
                raise abi.Unsupported(abi.EUNSUPPORTED, "block scales take int8 codes, no rotation, bf16 operands")
            lay = _LAYOUTS[layout]
            epi = _epilogue(epilogue)
            n_out = n // 2 if epi in (abi.EPI_SILU_GLU, abi.EPI_SITU_GLU) else n
            if a.numel() < m * k or c.numel() < m * n_out or int8.numel() < weight_offset + k * n:
                raise ValueError("a, c or the weight buffer smaller than m × k, m × n, k × n")
            if scales.dtype != torch.float32 or scales_offset % 4 or \
                    scales.numel() * 4 < scales_offset + 4 * (k // max(int(block), 1)) * n:
                raise ValueError("scales must be fp32, [k / block, n] after the offset (a multiple of 4 bytes)")
            secs = ctypes.c_double(0.0)
            # The first `cols` columns: the codes' and scales' strides (n, k) and C's (n_out) kept.
            if a.dtype == torch.float32 and not rounding:
                # The fp32 route on block scales (the reference's `blocks` pipeline on fp32 A).
                st = abi.load().sq8_linear_f32(self._h, _dev(a, "a"), k, 0, _dev(int8, "int8") + weight_offset,
                                               abi.INT8, lay, n if lay == abi.KN else k,
                                               _dev(scales, "scales") + scales_offset, abi.F32, abi.SCALE_BLOCKS,
                                               int(block), None if bias is None else _dev(bias, "bias"), epi,
                                               _dev(c, "c"), _cdtype(c.dtype), n_out, m, k, cols,
                                               None if settled else ctypes.byref(secs))
                abi.check(st, "sq8_linear_f32")
                return 0.0 if settled else secs.value
            st = abi.load().sq8_linear_blocks(self._h, _dev(a, "a"), _adtype(a), k, _dev(int8, "int8") + weight_offset,
                                              lay, n if lay == abi.KN else k, _dev(scales, "scales") + scales_offset,
                                              abi.F32, int(block), None if bias is None else _dev(bias, "bias"), epi,
                                              _dev(c, "c"), _cdtype(c.dtype), n_out, m, k, cols,
                                              None if settled else ctypes.byref(secs))
            abi.check(st, "sq8_linear_blocks")
            return 0.0 if settled else secs.value
        group = 0 if rotation is None else int(rotation[0] if isinstance(rotation, (tuple, list)) else rotation)
        if quantizing is not None or prequantized is not None:
            if fp8:
                raise abi.Unsupported(abi.EUNSUPPORTED, "W8A8 takes int8 weights")
            return self._w8a8_linear(a, int8, scales, per_column, c, m, k, n, weight_offset, scales_offset, group,
                                     prequantized, settled, layout, bias, epilogue)
        exact = a.dtype == torch.float32 and not rounding
        lay = _LAYOUTS[layout]
        wd = _wdtype(int8, fp8)
        epi = _epilogue(epilogue)
        n_out = n // 2 if epi in (abi.EPI_SILU_GLU, abi.EPI_SITU_GLU) else n
        if a.numel() < m * k or c.numel() < m * n_out:
            raise ValueError("a or c smaller than m × k / m × n")
        if int8.numel() * int8.element_size() < weight_offset + k * n:
            raise ValueError("the weight buffer is smaller than its offset + k × n")
        if scales.dtype != torch.float32 or scales.numel() * 4 < scales_offset + 4 * (n if per_column else 1):
            raise ValueError("scales must be fp32, n of them (or one) after the offset")
        if scales_offset % 4:
            raise ValueError("the scales' offset must be a multiple of 4 bytes")
        ldw = n if lay == abi.KN else k
        ldc = n_out
        if columns is not None and columns != n:
            # The first `columns` of W's columns (its layout's stride kept) into C's first columns.
            n = n_out = columns
        secs = ctypes.c_double(0.0)
        if exact:
            # The reference's `submit` on fp32 A: the fp32 route (three exact bf16 parts per value).
            st = abi.load().sq8_linear_f32(self._h, _dev(a, "a"), k, group, _dev(int8, "int8") + weight_offset, wd, lay,
                                           ldw, _dev(scales, "scales") + scales_offset, abi.F32,
                                           abi.SCALE_COLUMNS if per_column else abi.SCALE_TENSOR, 0,
                                           None if bias is None else _dev(bias, "bias"), epi,
                                           _dev(c, "c"), _cdtype(c.dtype), ldc, m, k, n,
                                           None if settled else ctypes.byref(secs))
            abi.check(st, "sq8_linear_f32")
            return 0.0 if settled else secs.value
        args = ((self._h, _dev(a, "a"), _adtype(a), k) + ((group,) if group else ()) +
                (_dev(int8, "int8") + weight_offset, wd, lay, ldw,
                 _dev(scales, "scales") + scales_offset, abi.SCALE_COLUMNS if per_column else abi.SCALE_TENSOR,
                 None if bias is None else _dev(bias, "bias"), epi,
                 _dev(c, "c"), _cdtype(c.dtype), ldc, m, k, n,
                 None if settled else ctypes.byref(secs)))
        name = "sq8_linear_rotated" if group else "sq8_linear"
        abi.check(getattr(abi.load(), name)(*args), name)
        return 0.0 if settled else secs.value

    def submit(self, a: torch.Tensor, *, int8: torch.Tensor, scales: torch.Tensor, per_column: bool,
               c: torch.Tensor, m: int, k: int, n: int, columns: int, weight_offset: int = 0, scales_offset: int = 0,
               block: Optional[int] = None, rotation=None, rounding=None, layout: str = "kn",
               bias: Optional[torch.Tensor] = None, epilogue=None, fp8: Optional[bool] = None) -> None:
        """`submit(a:int8:…:c:m:k:n:columns:)` (TensorGEMM.swift:292-360): the product on the first
        `columns` of C only, queued and not waited for — the caller computes the other columns
        meanwhile and synchronizes before reading C. `block`: block scales, as `linear`."""
        self.linear(a, int8=int8, scales=scales, per_column=per_column, c=c, m=m, k=k, n=n,
                    weight_offset=weight_offset, scales_offset=scales_offset, block=block, rotation=rotation,
                    rounding=rounding, settled=True, layout=layout, bias=bias, epilogue=epilogue, fp8=fp8,
                    columns=columns)

    def linear_bf16_weight(self, a: torch.Tensor, *, w: torch.Tensor, c: torch.Tensor, m: int, k: int, n: int,
                           weight_is_transposed: bool) -> float:
        """`linear(a:w:c:m:k:n:weightIsTransposed:)` (TensorGEMM.swift:236-254): C fp32 [m, n] = A [m, k] · W,
        W bf16 `[k, n]` when `weight_is_transposed` (the forge's layout), `[n, k]` otherwise, all row-major
        from offset 0. A fp32 (used whole: three exact bf16 parts) or bf16. Returns the GPU seconds."""
        if w.dtype != torch.bfloat16 or c.dtype != torch.float32:
            raise ValueError("w must be bf16 and c fp32")
        if a.numel() < m * k or w.numel() < k * n or c.numel() < m * n:
            raise ValueError("a, w or c smaller than m × k, k × n, m × n")
        secs = ctypes.c_double(0.0)
        st = abi.load().sq8_linear_bf16_weight(self._h, _dev(a, "a"), _adtype(a), k, _dev(w, "w"),
                                               abi.KN if weight_is_transposed else abi.NK,
                                               n if weight_is_transposed else k, _dev(c, "c"), n, m, k, n,
                                               ctypes.byref(secs))
        abi.check(st, "sq8_linear_bf16_weight")
        return secs.value

    def product_bf16_weight(self, x: torch.Tensor, w: torch.Tensor, *, layout: str = "nk",
                            out: Optional[torch.Tensor] = None, timed: bool = False):
        """y fp32 [m, n] = x · Wᵀ for W bf16 [n, k] (`"nk"`, nn.Linear) or x · W for W [k, n] (`"kn"`);
        x fp32 (used whole) or bf16. No scale, no bias: the bf16-weight product. Returns y (and the GPU
        seconds on the context's stream when `timed`)."""
        m, k = x.shape
        lay = _LAYOUTS[layout]
        if w.dtype != torch.bfloat16 or w.dim() != 2 or (w.shape[1] if lay == abi.NK else w.shape[0]) != k:
            raise ValueError(f"w must be bf16 [n, k] or [k, n] matching x [{m}, {k}]")
        n = w.shape[0] if lay == abi.NK else w.shape[1]
        if out is None:
            out = torch.empty((m, n), dtype=torch.float32, device=x.device)
        secs = ctypes.c_double(0.0)
        st = abi.load().sq8_linear_bf16_weight(self._h, _dev(x, "x"), _adtype(x), _row_major(x, "x"), _dev(w, "w"), lay,
                                               _row_major(w, "w"), _dev(out, "out"), _row_major(out, "out"), m, k, n,
                                               ctypes.byref(secs) if timed else None)
        abi.check(st, "sq8_linear_bf16_weight")
        return (out, secs.value) if timed else out

    def _w8a8_linear(self, a, int8, scales, per_column, c, m, k, n, weight_offset, scales_offset, group, prequantized,
                     settled, layout, bias, epilogue) -> float:
        lay = _LAYOUTS[layout]
        epi = _epilogue(epilogue)
        n_out = n // 2 if epi in (abi.EPI_SILU_GLU, abi.EPI_SITU_GLU) else n
        if c.numel() < m * n_out or int8.numel() < weight_offset + k * n:
            raise ValueError("c or the weight buffer too small")
        if scales.dtype != torch.float32 or scales.numel() * 4 < scales_offset + 4 * (n if per_column else 1):
            raise ValueError("scales must be fp32, n of them (or one) after the offset")
        ldw = n if lay == abi.KN else k
        secs = ctypes.c_double(0.0)
        common = (_dev(int8, "int8") + weight_offset, lay, ldw,
                  _dev(scales, "scales") + scales_offset, abi.SCALE_COLUMNS if per_column else abi.SCALE_TENSOR,
                  None if bias is None else _dev(bias, "bias"), epi,
                  _dev(c, "c"), _cdtype(c.dtype), n_out, m, k, n, None if settled else ctypes.byref(secs))
        if prequantized is not None:
            codes, sx = prequantized
            st = abi.load().sq8_linear_w8a8(self._h, _dev(codes, "codes"), _row_major(codes, "codes"),
                                            _dev(sx, "scales"), *common)
            abi.check(st, "sq8_linear_w8a8")
        else:
            st = abi.load().sq8_linear_quantized(self._h, _dev(a, "a"), _adtype(a), k, group, *common)
            abi.check(st, "sq8_linear_quantized")
        return 0.0 if settled else secs.value

    # ---- W8A8 (ComfyUI's int8_linear) ----------------------------------------------------------

    def quantize_rows(self, x: torch.Tensor, group: int = 0, *, codes: Optional[torch.Tensor] = None,
                      scales: Optional[torch.Tensor] = None):
        """Per-row int8 quantization of x [rows, k] (fp32 or bf16), rotated by groups of `group`
        first (0: none): (codes int8 [rows, k], scales fp32 [rows]) — W8A8.quantize's bits
        (TensorGEMMInt8.swift:198-221)."""
        if x.dim() != 2:
            raise ValueError("x must be 2-D [rows, k]")
        rows, k = x.shape
        if codes is None:
            codes = torch.empty((rows, k), dtype=torch.int8, device=x.device)
        if scales is None:
            scales = torch.empty(rows, dtype=torch.float32, device=x.device)
        if codes.dtype != torch.int8 or tuple(codes.shape) != (rows, k) or scales.dtype != torch.float32:
            raise ValueError("codes int8 [rows, k], scales fp32 [rows]")
        st = abi.load().sq8_quantize_rows(self._h, _dev(x, "x"), _adtype(x), _row_major(x, "x"), rows, k, int(group),
                                          _dev(codes, "codes"), _row_major(codes, "codes"), _dev(scales, "scales"))
        abi.check(st, "sq8_quantize_rows")
        return codes, scales

    def _w8a8_product(self, name, lead, m, k, w, scale, layout, bias, epilogue, out, out_dtype, timed, device):
        epi = _epilogue(epilogue)
        if isinstance(w, PackedWeight):
            if w.w_dtype != abi.INT8:
                raise ValueError("W8A8 takes int8 weights")
            lay, n, ldw, wptr = w.layout, w.n, w.k, _dev(w.data, "w")
            if w.k != k:
                raise ValueError(f"the packed weight has K = {w.k}, the activation {k}")
        else:
            if w.dtype != torch.int8 or w.dim() != 2:
                raise ValueError("W8A8 takes an int8 weight [n, k] (nk) or [k, n] (kn)")
            lay = _LAYOUTS[layout]
            n = w.shape[0] if lay == abi.NK else w.shape[1]
            ldw, wptr = _row_major(w, "w"), _dev(w, "w")
        glu = epi in (abi.EPI_SILU_GLU, abi.EPI_SITU_GLU)
        n_out = n // 2 if glu else n
        per_col = scale.numel() != 1
        if scale.dtype != torch.float32 or (per_col and scale.numel() != n):
            raise ValueError("scale must be fp32 with n entries (or one)")
        if out is None:
            out = torch.empty((m, n_out), dtype=out_dtype, device=device)
        secs = ctypes.c_double(0.0)
        st = getattr(abi.load(), name)(self._h, *lead, wptr, lay, ldw, _dev(scale, "scale"),
                                       abi.SCALE_COLUMNS if per_col else abi.SCALE_TENSOR,
                                       None if bias is None else _dev(bias, "bias"), epi, _dev(out, "out"),
                                       _cdtype(out.dtype), _row_major(out, "out"), m, k, n,
                                       ctypes.byref(secs) if timed else None)
        abi.check(st, name)
        return (out, secs.value) if timed else out

    def product_w8a8(self, codes: torch.Tensor, sx: torch.Tensor, w, scale: torch.Tensor, *, layout: str = "nk",
                     bias: Optional[torch.Tensor] = None, epilogue=None, out: Optional[torch.Tensor] = None,
                     out_dtype: torch.dtype = torch.bfloat16, timed: bool = False):
        """act(float(codes · qᵀ) · (s_x · s_w) + b) on an activation already quantized (codes int8
        [m, k], sx fp32 [m]); W int8 [n, k] (`nk`), [k, n] (`kn`) or a PackedWeight."""
        if codes.dtype != torch.int8 or sx.dtype != torch.float32:
            raise ValueError("codes int8 [m, k], sx fp32 [m]")
        m, k = codes.shape
        return self._w8a8_product("sq8_linear_w8a8", (_dev(codes, "codes"), _row_major(codes, "codes"), _dev(sx, "sx")),
                                  m, k, w, scale, layout, bias, epilogue, out, out_dtype, timed, codes.device)

    def product_quantized(self, x: torch.Tensor, w, scale: torch.Tensor, *, group: int = 0, layout: str = "nk",
                          bias: Optional[torch.Tensor] = None, epilogue=None, out: Optional[torch.Tensor] = None,
                          out_dtype: torch.dtype = torch.bfloat16, timed: bool = False):
        """The W8A8 route whole: x (fp32 or bf16 [m, k]) quantized per row (rotated by `group`
        first), then the int8 × int8 product as `product_w8a8`."""
        m, k = x.shape
        return self._w8a8_product("sq8_linear_quantized", (_dev(x, "x"), _adtype(x), _row_major(x, "x"), int(group)),
                                  m, k, w, scale, layout, bias, epilogue, out, out_dtype, timed, x.device)

    # ---- staging -----------------------------------------------------------------------------

    def pack(self, w: torch.Tensor, *, layout: str = "nk", glu: bool = False,
             fp8: Optional[bool] = None) -> PackedWeight:
        """Stages codes W ([n, k] for "nk", [k, n] for "kn") into the packed layout, once
        (Artifact.stageInt8's place, Sources/Siliconed/Artifact.swift:755-774)."""
        lay = _LAYOUTS[layout]
        wd = _wdtype(w, fp8)
        if w.dim() != 2:
            raise ValueError("w must be 2-D")
        n, k = (w.shape[0], w.shape[1]) if lay == abi.NK else (w.shape[1], w.shape[0])
        if glu and n % 2:
            raise ValueError("a GLU weight has an even number of columns")
        size = abi.load().sq8_packed_bytes(k, n, int(glu))
        out = torch.empty(max(size, 1), dtype=torch.uint8, device=w.device)
        st = abi.load().sq8_pack_weight(self._h, _dev(w, "w"), lay, _row_major(w, "w"), k, n, int(glu), out.data_ptr())
        abi.check(st, "sq8_pack_weight")
        return PackedWeight(out, k, n, glu, wd)

    def pack_blocks(self, w: torch.Tensor, scale: torch.Tensor, block: int, *, layout: str = "nk",
                    glu: bool = False) -> PackedBlocks:
        """Stages block-scaled int8 codes W ([n, k] "nk" with scales [n, k/block]; [k, n] "kn" with
        scales [k/block, n]; scales fp32, bf16 or fp16) into the packed Q8 layout, once."""
        lay = _LAYOUTS[layout]
        if w.dtype != torch.int8 or w.dim() != 2:
            raise ValueError("block scales take int8 codes, 2-D")
        n, k = (w.shape[0], w.shape[1]) if lay == abi.NK else (w.shape[1], w.shape[0])
        if block <= 0 or k % block:
            raise ValueError(f"k = {k} is not a multiple of the block {block}")
        _block_scales(scale, lay, n, k, block, _row_major(w, "w"))
        size = abi.load().sq8_packed_blocks_bytes(k, n, int(glu))
        if size < 0:
            raise ValueError("a GLU weight has an even number of columns")
        out = torch.empty(max(size, 1), dtype=torch.uint8, device=w.device)
        st = abi.load().sq8_pack_blocks(self._h, _dev(w, "w"), lay, _row_major(w, "w"), _dev(scale, "scale"),
                                        _SCALE_DTYPES[scale.dtype], int(block), k, n, int(glu), out.data_ptr())
        abi.check(st, "sq8_pack_blocks")
        return PackedBlocks(out, k, n, glu, int(block))

    def product_blocks(self, x: torch.Tensor, w, scale: Optional[torch.Tensor] = None, block: int = 32, *,
                       layout: str = "nk", bias: Optional[torch.Tensor] = None, epilogue=None,
                       out: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.bfloat16,
                       timed: bool = False, rounding: bool = True):
        """y = act(x · Wᵀ + b), W[n, k] = q · s[block of k, n] (GGUF Q8_0: block 32): x [m, k] bf16
        (or fp32: rounded, or with `rounding=False` used whole, the fp32 route); W int8 codes [n, k]
        ("nk", scales [n, k/block]) or [k, n] ("kn", scales [k/block, n]), or a PackedBlocks (scale and
        block from it)."""
        epi = _epilogue(epilogue)
        m, k = x.shape
        if isinstance(w, PackedBlocks):
            if w.k != k:
                raise ValueError(f"x [{m}, {k}] and the packed weight disagree on K ({w.k})")
            if w.glu != (epi in (abi.EPI_SILU_GLU, abi.EPI_SITU_GLU)):
                raise ValueError("a weight packed for a GLU epilogue serves GLU epilogues only, and only those")
            lay, n, ldw, wptr, sptr, sdt, block = w.layout, w.n, w.k, _dev(w.data, "w"), None, abi.F32, w.block
        else:
            lay = _LAYOUTS[layout]
            if w.dtype != torch.int8 or w.dim() != 2:
                raise ValueError("block scales take int8 codes, 2-D")
            n = w.shape[0] if lay == abi.NK else w.shape[1]
            if (w.shape[1] if lay == abi.NK else w.shape[0]) != k:
                raise ValueError(f"x [{m}, {k}] and w {tuple(w.shape)} ({layout}) disagree on K")
            if block <= 0 or k % block:
                raise ValueError(f"k = {k} is not a multiple of the block {block}")
            _block_scales(scale, lay, n, k, block, _row_major(w, "w"))
            ldw, wptr, sptr, sdt = _row_major(w, "w"), _dev(w, "w"), _dev(scale, "scale"), _SCALE_DTYPES[scale.dtype]
        n_out = n // 2 if epi in (abi.EPI_SILU_GLU, abi.EPI_SITU_GLU) else n
        if out is None:
            out = torch.empty((m, n_out), dtype=out_dtype, device=x.device)
        secs = ctypes.c_double(0.0)
        if not rounding and x.dtype == torch.float32:
            st = abi.load().sq8_linear_f32(self._h, _dev(x, "x"), _row_major(x, "x"), 0, wptr, abi.INT8, lay, ldw,
                                           sptr, sdt, abi.SCALE_BLOCKS, int(block),
                                           None if bias is None else _dev(bias, "bias"), epi, _dev(out, "out"),
                                           _cdtype(out.dtype), _row_major(out, "out"), m, k, n,
                                           ctypes.byref(secs) if timed else None)
            abi.check(st, "sq8_linear_f32")
            return (out, secs.value) if timed else out
        st = abi.load().sq8_linear_blocks(self._h, _dev(x, "x"), _adtype(x), _row_major(x, "x"), wptr, lay, ldw, sptr,
                                          sdt, int(block), None if bias is None else _dev(bias, "bias"), epi,
                                          _dev(out, "out"), _cdtype(out.dtype), _row_major(out, "out"), m, k, n,
                                          ctypes.byref(secs) if timed else None)
        abi.check(st, "sq8_linear_blocks")
        return (out, secs.value) if timed else out

    # ---- tensor-level operations ---------------------------------------------------------------

    def product(self, x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, *, layout: str = "nk",
                bias: Optional[torch.Tensor] = None, epilogue=None, out: Optional[torch.Tensor] = None,
                out_dtype: torch.dtype = torch.bfloat16, fp8: Optional[bool] = None,
                timed: bool = False, rotation: int = 0, rounding: bool = True):
        """y = act(s ⊙ (x · Wᵀ) + b) for x [m, k] and W [n, k] (`layout="nk"`, nn.Linear) or
        [k, n] (`"kn"`, the map's). `rotation` = G: a convrot weight, x rotated by groups of G
        first (y = act(s ⊙ ((x·R) · qᵀ) + b)). An fp32 x is rounded to bf16 first (`rounding`, the
        reference's submitRounded), or with `rounding=False` used whole: the fp32 route (sq8_linear_f32;
        with a `rotation`, x rotated in fp32 first). Returns y (and the GPU seconds when `timed`)."""
        exact = not rounding and x.dtype == torch.float32
        epi = _epilogue(epilogue)
        m, k = x.shape
        if isinstance(w, PackedWeight):
            lay, wd, n, ldw, wptr = w.layout, w.w_dtype, w.n, w.k, _dev(w.data, "w")
            if w.k != k:
                raise ValueError(f"x [{m}, {k}] and the packed weight disagree on K ({w.k})")
            if w.glu != (epi in (abi.EPI_SILU_GLU, abi.EPI_SITU_GLU)):
                raise ValueError("a weight packed for a GLU epilogue serves GLU epilogues only, and only those")
        else:
            lay = _LAYOUTS[layout]
            wd = _wdtype(w, fp8)
            if w.dim() != 2:
                raise ValueError("w must be 2-D")
            n = w.shape[0] if lay == abi.NK else w.shape[1]
            if (w.shape[1] if lay == abi.NK else w.shape[0]) != k:
                raise ValueError(f"x [{m}, {k}] and w {tuple(w.shape)} ({layout}) disagree on K")
            ldw, wptr = _row_major(w, "w"), _dev(w, "w")
        glu = epi in (abi.EPI_SILU_GLU, abi.EPI_SITU_GLU)
        if glu and n % 2:
            raise ValueError("a GLU epilogue needs an even number of weight columns")
        n_out = n // 2 if glu else n
        per_col = scale.numel() != 1
        if scale.dtype != torch.float32 or (per_col and scale.numel() != n):
            raise ValueError("scale must be fp32 with n entries (or one)")
        if bias is not None and (bias.dtype != torch.float32 or bias.numel() != n):
            raise ValueError("bias must be fp32 with n entries")
        if out is None:
            out = torch.empty((m, n_out), dtype=out_dtype, device=x.device)
        elif tuple(out.shape) != (m, n_out):
            raise ValueError("out has the wrong shape")
        secs = ctypes.c_double(0.0)
        if exact:
            st = abi.load().sq8_linear_f32(self._h, _dev(x, "x"), _row_major(x, "x"), int(rotation), wptr, wd, lay,
                                           ldw, _dev(scale, "scale"), abi.F32,
                                           abi.SCALE_COLUMNS if per_col else abi.SCALE_TENSOR, 0,
                                           None if bias is None else _dev(bias, "bias"), epi, _dev(out, "out"),
                                           _cdtype(out.dtype), _row_major(out, "out"), m, k, n,
                                           ctypes.byref(secs) if timed else None)
            abi.check(st, "sq8_linear_f32")
            return (out, secs.value) if timed else out
        args = ((self._h, _dev(x, "x"), _adtype(x), _row_major(x, "x")) + ((int(rotation),) if rotation else ()) +
                (wptr, wd, lay, ldw,
                 _dev(scale, "scale"), abi.SCALE_COLUMNS if per_col else abi.SCALE_TENSOR,
                 None if bias is None else _dev(bias, "bias"), epi,
                 _dev(out, "out"), _cdtype(out.dtype), _row_major(out, "out"), m, k, n,
                 ctypes.byref(secs) if timed else None))
        name = "sq8_linear_rotated" if rotation else "sq8_linear"
        abi.check(getattr(abi.load(), name)(*args), name)
        return (out, secs.value) if timed else out

    def product_qkv(self, x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, *, layout: str = "nk",
                    bias: Optional[torch.Tensor] = None, head_dim: int = 0,
                    out_dtype: torch.dtype = torch.bfloat16, fp8: Optional[bool] = None, out=None):
        """Fused QKV: W of 3·d output channels; returns (q, k, v), each [m, d] (head_dim 0) or
        [d/head_dim, m, head_dim]. `out`: three preallocated tensors of that shape (contiguous)."""
        m, k = x.shape
        if isinstance(w, PackedWeight):
            lay, wd, n, ldw, wptr = w.layout, w.w_dtype, w.n, w.k, _dev(w.data, "w")
        else:
            lay = _LAYOUTS[layout]
            wd = _wdtype(w, fp8)
            n = w.shape[0] if lay == abi.NK else w.shape[1]
            ldw, wptr = _row_major(w, "w"), _dev(w, "w")
        if n % 3:
            raise ValueError("a fused QKV weight has 3·d output channels")
        d = n // 3
        shape = (m, d) if head_dim == 0 else (d // head_dim, m, head_dim)
        if out is None:
            q, kk, v = (torch.empty(shape, dtype=out_dtype, device=x.device) for _ in range(3))
        else:
            q, kk, v = out
            for t in out:
                if tuple(t.shape) != shape or not t.is_contiguous() or t.dtype not in (torch.bfloat16, torch.float32):
                    raise ValueError(f"QKV outputs must be contiguous {shape} bf16/fp32 tensors")
            out_dtype = q.dtype
        per_col = scale.numel() != 1
        st = abi.load().sq8_linear_qkv(
            self._h, _dev(x, "x"), _adtype(x), _row_major(x, "x"),
            wptr, wd, lay, ldw,
            _dev(scale, "scale"), abi.SCALE_COLUMNS if per_col else abi.SCALE_TENSOR,
            None if bias is None else _dev(bias, "bias"),
            q.data_ptr(), kk.data_ptr(), v.data_ptr(), _cdtype(out_dtype), d, head_dim, m, k, d, None)
        abi.check(st, "sq8_linear_qkv")
        return q, kk, v

    # ---- the DiT block's elementwise passes ----------------------------------------------------------

    def norm_modulate(self, x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                      eps: float = 1e-6, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """bf16(((x·r)·w)·(1 + scale) + shift), r = 1/sqrt(mean(x²) + eps) per row of fp32 x
        (`norm_modulate_rounded`, ElementwiseGPUMoss.swift:45-91)."""
        rows, cols = x.shape
        for t, what in ((x, "x"), (w, "w"), (scale, "scale"), (shift, "shift")):
            if t.dtype != torch.float32:
                raise ValueError(f"{what} must be fp32")
        for t, what in ((w, "w"), (scale, "scale"), (shift, "shift")):
            if t.numel() != cols or not t.is_contiguous():
                raise ValueError(f"{what} must be {cols} contiguous values")
        if out is None:
            out = torch.empty((rows, cols), dtype=torch.bfloat16, device=x.device)
        st = abi.load().sq8_norm_modulate(self._h, _dev(x, "x"), _row_major(x, "x"), _dev(w, "w"), _dev(scale, "scale"),
                                          _dev(shift, "shift"), float(eps), _dev(out, "out"), _row_major(out, "out"),
                                          rows, cols)
        abi.check(st, "sq8_norm_modulate")
        return out

    def _norm_args(self, x, w, scale, shift, y_out):
        if x.dtype != torch.float32 or x.dim() != 2:
            raise ValueError("x must be fp32 [rows, cols]")
        rows, cols = x.shape
        for t, name in ((w, "w"), (scale, "scale"), (shift, "shift")):
            if t.dtype != torch.float32 or t.numel() != cols or not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous fp32 [cols]")
        if y_out is not None and (y_out.dtype != torch.float32 or tuple(y_out.shape) != (rows, cols)):
            raise ValueError("y_out must be fp32 [rows, cols]")
        return rows, cols

    def norm_modulate_rotated(self, x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                              eps: float, group: int, *, out: Optional[torch.Tensor] = None,
                              y_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The modulated RMSNorm's row y, rotated by `group` and rounded to bf16: a convrot product's
        operand in one pass (y itself into `y_out` when given)."""
        rows, cols = self._norm_args(x, w, scale, shift, y_out)
        if out is None:
            out = torch.empty((rows, cols), dtype=torch.bfloat16, device=x.device)
        st = abi.load().sq8_norm_modulate_rotated(
            self._h, _dev(x, "x"), _row_major(x, "x"), _dev(w, "w"), _dev(scale, "scale"), _dev(shift, "shift"), eps,
            int(group), _dev(out, "out"), _row_major(out, "out"),
            None if y_out is None else _dev(y_out, "y_out"), 0 if y_out is None else _row_major(y_out, "y_out"), rows, cols)
        abi.check(st, "sq8_norm_modulate_rotated")
        return out

    def norm_modulate_quantized(self, x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                                eps: float, group: int = 0, *, codes: Optional[torch.Tensor] = None,
                                scales: Optional[torch.Tensor] = None, y_out: Optional[torch.Tensor] = None):
        """The modulated RMSNorm's row y, rotated by `group` (0: none) and quantized per row: a W8A8
        product's operand (codes int8 [rows, cols], scales fp32 [rows]) in one pass."""
        rows, cols = self._norm_args(x, w, scale, shift, y_out)
        if codes is None:
            codes = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
        if scales is None:
            scales = torch.empty(rows, dtype=torch.float32, device=x.device)
        st = abi.load().sq8_norm_modulate_quantized(
            self._h, _dev(x, "x"), _row_major(x, "x"), _dev(w, "w"), _dev(scale, "scale"), _dev(shift, "shift"), eps,
            int(group), _dev(codes, "codes"), _row_major(codes, "codes"), _dev(scales, "scales"),
            None if y_out is None else _dev(y_out, "y_out"), 0 if y_out is None else _row_major(y_out, "y_out"), rows, cols)
        abi.check(st, "sq8_norm_modulate_quantized")
        return codes, scales

    def product_w8a8_qkv(self, codes: torch.Tensor, sx: torch.Tensor, w, scale: torch.Tensor, *,
                         bias: Optional[torch.Tensor] = None, head_dim: int = 0, out=None,
                         out_dtype: torch.dtype = torch.bfloat16):
        """The W8A8 fused QKV: (q, k, v), each [m, d] (head_dim 0) or [d/head_dim, m, head_dim]."""
        m, k = codes.shape
        if isinstance(w, PackedWeight):
            lay, n, ldw, wptr = w.layout, w.n, w.k, _dev(w.data, "w")
        else:
            lay, n, ldw, wptr = abi.NK, w.shape[0], _row_major(w, "w"), _dev(w, "w")
        if n % 3:
            raise ValueError("a fused QKV weight has 3·d columns")
        d = n // 3
        shape = (m, d) if head_dim == 0 else (d // head_dim, m, head_dim)
        if out is None:
            out = tuple(torch.empty(shape, dtype=out_dtype, device=codes.device) for _ in range(3))
        per_col = scale.numel() != 1
        st = abi.load().sq8_linear_w8a8_qkv(
            self._h, _dev(codes, "codes"), _row_major(codes, "codes"), _dev(sx, "sx"), wptr, lay, ldw,
            _dev(scale, "scale"), abi.SCALE_COLUMNS if per_col else abi.SCALE_TENSOR,
            None if bias is None else _dev(bias, "bias"), _dev(out[0], "q"), _dev(out[1], "k"), _dev(out[2], "v"),
            _cdtype(out_dtype), d if head_dim == 0 else 0, head_dim, m, k, d, None)
        abi.check(st, "sq8_linear_w8a8_qkv")
        return out

    def product_residual(self, x: torch.Tensor, a: torch.Tensor, w, scale: torch.Tensor, *, layout: str = "nk",
                         bias: Optional[torch.Tensor] = None, gate: Optional[torch.Tensor] = None,
                         fp8: Optional[bool] = None) -> torch.Tensor:
        """x += gate ⊙ (s ⊙ (a · Wᵀ) + b) in place (x fp32 [m, n], the residual stream), one pass."""
        m, k = a.shape
        if isinstance(w, PackedWeight):
            lay, wd, n, ldw, wptr = w.layout, w.w_dtype, w.n, w.k, _dev(w.data, "w")
        else:
            lay, wd = _LAYOUTS[layout], _wdtype(w, fp8)
            n = w.shape[0] if lay == abi.NK else w.shape[1]
            ldw, wptr = _row_major(w, "w"), _dev(w, "w")
        if x.dtype != torch.float32 or tuple(x.shape) != (m, n):
            raise ValueError("x must be the fp32 residual stream [m, n]")
        st = abi.load().sq8_linear_residual(
            self._h, _dev(a, "a"), _adtype(a), _row_major(a, "a"), wptr, wd, lay, ldw,
            _dev(scale, "scale"), abi.SCALE_COLUMNS if scale.numel() != 1 else abi.SCALE_TENSOR,
            None if bias is None else _dev(bias, "bias"), None if gate is None else _dev(gate, "gate"),
            _dev(x, "x"), _row_major(x, "x"), m, k, n, None)
        abi.check(st, "sq8_linear_residual")
        return x

    def product_w8a8_residual(self, x: torch.Tensor, codes: torch.Tensor, sx: torch.Tensor, w, scale: torch.Tensor, *,
                              layout: str = "nk", bias: Optional[torch.Tensor] = None,
                              gate: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x += gate ⊙ (float(codes · qᵀ) · (s_x · s_w) + b) in place, one pass."""
        m, k = codes.shape
        if isinstance(w, PackedWeight):
            lay, n, ldw, wptr = w.layout, w.n, w.k, _dev(w.data, "w")
        else:
            lay = _LAYOUTS[layout]
            n = w.shape[0] if lay == abi.NK else w.shape[1]
            ldw, wptr = _row_major(w, "w"), _dev(w, "w")
        if x.dtype != torch.float32 or tuple(x.shape) != (m, n):
            raise ValueError("x must be the fp32 residual stream [m, n]")
        st = abi.load().sq8_linear_w8a8_residual(
            self._h, _dev(codes, "codes"), _row_major(codes, "codes"), _dev(sx, "sx"), wptr, lay, ldw,
            _dev(scale, "scale"), abi.SCALE_COLUMNS if scale.numel() != 1 else abi.SCALE_TENSOR,
            None if bias is None else _dev(bias, "bias"), None if gate is None else _dev(gate, "gate"),
            _dev(x, "x"), _row_major(x, "x"), m, k, n, None)
        abi.check(st, "sq8_linear_w8a8_residual")
        return x

    def rms_rows(self, t: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
        """In place: each row of the bf16 tensor t (last dimension ≤ 256, rows contiguous) →
        bf16((t·r)·w) — the per-head RMSNorm of q and k."""
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError("t must be bf16 with contiguous rows")
        cols = t.shape[-1]
        rows = t.numel() // cols
        ld = t.stride(-2) if t.dim() > 1 else cols
        if t.dim() > 2 and not t.is_contiguous():
            raise ValueError("t must be contiguous beyond its rows")
        if w.dtype != torch.float32 or w.numel() != cols:
            raise ValueError(f"w must be {cols} fp32 values")
        abi.check(abi.load().sq8_rms_rows(self._h, _dev(t, "t"), ld, rows, cols, _dev(w, "w"), float(eps)), "sq8_rms_rows")
        return t

    def gated_residual(self, x: torch.Tensor, y: torch.Tensor, gate: Optional[torch.Tensor] = None) -> torch.Tensor:
        """In place: x += gate ⊙ y (x fp32 [rows, cols], y bf16 or fp32, gate fp32 [cols])."""
        if x.dtype != torch.float32 or x.shape != y.shape:
            raise ValueError("x must be fp32 and y of its shape")
        rows, cols = x.shape
        if gate is not None and (gate.dtype != torch.float32 or gate.numel() != cols or not gate.is_contiguous()):
            raise ValueError(f"gate must be {cols} contiguous fp32 values")
        st = abi.load().sq8_gated_residual(self._h, _dev(x, "x"), _row_major(x, "x"), _dev(y, "y"), _adtype(y),
                                           _row_major(y, "y"), None if gate is None else _dev(gate, "gate"), rows, cols)
        abi.check(st, "sq8_gated_residual")
        return x

    def dequantize(self, codes: torch.Tensor, scale: Optional[torch.Tensor] = None, *,
                   layout: int = abi.SCALE_COLUMNS, block_rows: int = 0, first_row: int = 0,
                   fp8: Optional[bool] = None) -> torch.Tensor:
        """Float(q)·s on the device (Widen.dequantize, Widen.swift:129-271); codes [rows, columns]."""
        wd = _wdtype(codes, fp8)
        codes2 = codes if codes.dim() == 2 else codes.reshape(1, -1)
        rows, cols = codes2.shape
        if not codes2.is_contiguous():
            raise ValueError("codes must be contiguous")
        out = torch.empty((rows, cols), dtype=torch.float32, device=codes.device)
        sd = 0
        if scale is not None:
            sd = {torch.float32: abi.F32, torch.bfloat16: abi.BF16, torch.float16: abi.F16}.get(scale.dtype)
            if sd is None:
                raise ValueError("scales are fp32, bf16 or fp16")
        st = abi.load().sq8_dequantize(self._h, codes2.data_ptr(), wd, rows, cols,
                                       None if scale is None else _dev(scale, "scale"), sd, layout, block_rows,
                                       first_row, out.data_ptr())
        abi.check(st, "sq8_dequantize")
        return out.reshape(codes.shape)

    def rotate(self, x: torch.Tensor, group: int, *, out: Optional[torch.Tensor] = None,
               out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """x·R by groups of `group` along the rows of x [rows, k] (fp32 or bf16): the activation's
        convrot rotation (rotate_groups, TensorGEMM.swift:181-201), fp32 butterflies, the result
        rounded to bf16 (`out_dtype`) or kept fp32. `out` may be x itself (same dtype)."""
        if x.dim() != 2:
            raise ValueError("x must be 2-D [rows, k]")
        rows, k = x.shape
        if out is None:
            out = torch.empty((rows, k), dtype=out_dtype, device=x.device)
        elif tuple(out.shape) != (rows, k):
            raise ValueError("out has the wrong shape")
        st = abi.load().sq8_rotate_groups(self._h, _dev(x, "x"), _adtype(x), _row_major(x, "x"),
                                          _dev(out, "out"), _cdtype(out.dtype), _row_major(out, "out"), rows, k,
                                          int(group))
        abi.check(st, "sq8_rotate_groups")
        return out

    def dequantize_rotated(self, codes: torch.Tensor, group: int, scale: torch.Tensor) -> torch.Tensor:
        """Float(H·q)·(s/√G) of int8 codes [k, n] rotated along k (Widen.dequantizeRotated,
        Widen.swift:374-428): fp32 [k, n]. `scale` fp32/bf16/fp16, n of them or one."""
        if codes.dtype != torch.int8 or codes.dim() != 2:
            raise ValueError("codes must be int8 [k, n]")
        k, n = codes.shape
        sd = {torch.float32: abi.F32, torch.bfloat16: abi.BF16, torch.float16: abi.F16}.get(scale.dtype)
        if sd is None:
            raise ValueError("scales are fp32, bf16 or fp16")
        if scale.numel() not in (1, n):
            raise ValueError("scale: n of them, or one")
        out = torch.empty((k, n), dtype=torch.float32, device=codes.device)
        st = abi.load().sq8_dequantize_rotated(self._h, _dev(codes, "codes"), _row_major(codes, "codes"), k, n,
                                               int(group), _dev(scale, "scale"), sd,
                                               abi.SCALE_COLUMNS if scale.numel() == n and n != 1 else abi.SCALE_TENSOR,
                                               _dev(out, "out"), n)
        abi.check(st, "sq8_dequantize_rotated")
        return out

    def round_bf16(self, x: torch.Tensor) -> torch.Tensor:
        """fp32 → bf16 nearest-even (TensorGEMMBF16.swift:41-48)."""
        if x.dtype != torch.float32 or not x.is_contiguous():
            raise ValueError("x must be contiguous fp32")
        y = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
        st = abi.load().sq8_round_bf16(self._h, x.data_ptr(), y.data_ptr(), x.numel())
        abi.check(st, "sq8_round_bf16")
        return y


_contexts: dict = {}


def context(device: Optional[int] = None) -> TensorGEMM:
    """The default context of a device (on torch's current stream at creation)."""
    if device is None:
        device = torch.cuda.current_device()
    ctx = _contexts.get(device)
    if ctx is None:
        ctx = TensorGEMM.make(device)
        if ctx is None:
            raise abi.Unsupported(abi.ENODEVICE, f"device {device} is not a gfx950")
        _contexts[device] = ctx
    ctx.set_stream(torch.cuda.current_stream(device))
    return ctx


def linear(x, w, scale, **kw):
    """Functional form of `TensorGEMM.product` on the current device and stream."""
    return context(x.device.index).product(x, w, scale, **kw)


def linear_qkv(x, w, scale, **kw):
    return context(x.device.index).product_qkv(x, w, scale, **kw)


def pack(w, **kw):
    return context(w.device.index).pack(w, **kw)


def dequantize(codes, scale=None, **kw):
    return context(codes.device.index).dequantize(codes, scale, **kw)


def rotate(x, group, **kw):
    return context(x.device.index).rotate(x, group, **kw)


def dequantize_rotated(codes, group, scale):
    return context(codes.device.index).dequantize_rotated(codes, group, scale)


def round_bf16(x):
    return context(x.device.index).round_bf16(x)
