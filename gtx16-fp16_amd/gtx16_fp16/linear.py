"""nn.Linear replacement that stores fp16 weights and computes with the gfx950 kernels.

Mirrors the reference's src/gtx16_fp16/linear.py: same class, buffers, dtype rules and fallbacks.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _clib
from .kernels import SKINNY_MAX_M, PreparedCall, split_buffers, stream_handle
from .ops import (STRIPS_MAX_M, _is_target, _sm_count, is_affected, mm_t, mm_t_prepacked, pack_decode_weight,
                  pack_weight, prepacked_route, skinny_strips, supported, tensor_version)


class FastLinear(nn.Module):
    """Drop-in for ``nn.Linear`` at inference time, backed by the gfx950 kernels (the reference's
    class of the same name, linear.py:12-76, keeps the same buffers and rules).

    State: ``weight_t`` is the weight transposed to [in_features, out_features] and rounded once to
    fp16 (nearest-even); ``bias`` stays fp32. Those two buffers are the whole state_dict.

    Which kernel a call reaches depends on its row count M (all leading dimensions flattened):
    M <= 8 goes to the skinny GEMV, which multiplies the activations exactly as given (fp32 or fp16)
    in fp32 arithmetic; M > 8 goes to the MFMA GEMM, which first rounds each activation row to fp16
    after dividing it by a power of two when its largest magnitude exceeds 1024, accumulates in
    fp32, and multiplies the power of two back in. fp32 and fp16 inputs give outputs of their own
    dtype; any other input dtype is computed as fp32 and returns fp32. Inputs that need autograd,
    and shapes the kernels cannot take, are computed by ``F.linear`` instead.

    On the tile-packed GEMM route (large M) the layer also builds, on first use, a copy of its
    weight in the GEMM's packed layout and keeps it outside the state_dict; it is rebuilt whenever
    ``weight_t`` is replaced, moved or modified in place through torch. That spends one more fp16
    copy of the weight (the layer then holds as many bytes as the fp32 ``nn.Linear`` it replaced)
    to save the GEMM's transposing LDS reads; ``prepack_weight = False`` (on the class or an
    instance) turns it off.

    Two more caches are opt-in, because each trades memory or a staleness risk for speed:

    * ``share_cast = True``: large-batch layers called one after another with the same input tensor
      (a transformer's Q, K and V projections) on one stream reuse the first call's rowscale cast.
      A cast is reused only while the input is the same live tensor with the same torch version
      counter; writes that bypass torch's counter (a custom kernel writing through ``data_ptr()``,
      ``x.data.copy_()``, a serving stack refilling the buffer in place) are not seen and would
      make the next layer read a stale cast. Inputs created under ``torch.inference_mode()`` carry
      no version counter and are never shared. ``ops.release_cast_cache()`` frees the cached cast.
    * ``prepack_decode = True``: token-by-token calls (fp32 or fp16 activations, M <= 4 where the
      library's rule expects a gain) run on a second copy of the weight in a strip-major decode
      layout (8 columns by all of K per strip), built on the first such call and rebuilt whenever
      ``weight_t`` changes: one workgroup per strip needs no split of K and no exchange of partial
      sums between workgroups (4096 x 4096 at M = 1: 8.7 -> 7.3 us; 1024 x 1024: 5.0 -> 3.0 us).
      Same semantics as the skinny path, with the fp32 additions in another order. It costs one
      more fp16 copy of the weight (with the packed copy: three fp16 copies per layer, 1.5x the
      bytes of the fp32 layer).

    Neither copy is built while the current stream is being captured into a graph (the call takes
    the route on ``weight_t`` instead); a copy is built eagerly, and the device is synchronised
    around the build, so the copy is complete before any stream reads it and the one it replaces
    is no longer read when it is freed. A ``weight_t`` that is an inference tensor (made under
    ``torch.inference_mode()``) has no version counter: in-place writes to it are not seen (replace
    the tensor, or call ``release_copies()``).
    """

    prepack_weight = True
    # opt-in: a second fp16 copy of the weight in the decode layout (see the class docstring)
    prepack_decode = False
    # opt-in: large-batch calls whose input is the same unmodified tensor as the previous such call
    # on the stream (a transformer's Q, K and V projections) reuse that call's rowscale cast
    share_cast = False

    def __init__(self, in_features: int, out_features: int, bias: bool = True, device=None):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        # (M, device index, prepack_decode) -> (PreparedCall of the split kernel or None, ksplit,
        # (partial, counter) bytes, weight pointer, bias pointer, PreparedCall of the decode-layout
        # kernel or None) for the token-by-token fast path; None in the first field when the weight or
        # bias the pointers name cannot be handed to the kernel (the call then takes the general
        # path); the last field is set where the decode layout serves the call.
        self._skinny: dict = {}
        # decode-layout weight for the token-by-token route and the (pointer, version, device) of
        # weight_t it was built from
        self._wd: torch.Tensor | None = None
        self._wd_key: tuple | None = None
        self._wd_ptr = 0
        # prepacked weight for the large-GEMM route and the (pointer, version, device) of weight_t it
        # was built from
        self._wp: torch.Tensor | None = None
        self._wp_key: tuple | None = None
        self.register_buffer("weight_t", torch.empty(in_features, out_features, dtype=torch.float16, device=device))
        self.register_buffer("bias", torch.empty(out_features, dtype=torch.float32, device=device) if bias else None)

    @classmethod
    def from_linear(cls, lin: nn.Linear) -> "FastLinear":
        """Copy ``lin``: weight transposed and rounded to fp16 (nearest-even), bias as fp32
        (linear.py:30-37)."""
        m = cls(lin.in_features, lin.out_features, lin.bias is not None, device=lin.weight.device)
        with torch.no_grad():
            m.weight_t.copy_(lin.weight.detach().t().to(torch.float16))
            if lin.bias is not None:
                m.bias.copy_(lin.bias.detach().float())
        return m

    @property
    def weight(self) -> torch.Tensor:
        """[out_features, in_features] view of ``weight_t``, for callers that inspect a linear
        layer's ``.weight`` (its shape, device or dtype) as they would on nn.Linear."""
        return self.weight_t.t()

    def _decode_entry(self, M: int, dev: torch.device):
        key = (M, dev.index, self.prepack_decode)
        w, b = self.weight_t, self.bias
        bptr = None if b is None else b.data_ptr()
        entry = self._skinny.get(key)
        if entry is None or entry[3] != w.data_ptr() or entry[4] != bptr:
            # (re)validated whenever weight_t or bias is a different tensor, e.g. after .to() or
            # .half() (which turns the bias fp16: the kernel reads an fp32 bias)
            K, N = self.in_features, self.out_features
            ok = (w.dtype == torch.float16 and w.is_contiguous() and w.device == dev and K % 8 == 0
                  and N % 8 == 0 and w.data_ptr() % 16 == 0 and _is_target(dev.index or 0)
                  and (b is None or (b.dtype == torch.float32 and b.device == dev and b.is_contiguous()
                                     and b.numel() == N)))
            pl, ksplit, sizes, pls = None, 0, (0, 0), None
            if ok:
                lib = _clib.load()
                # the split kernel on weight_t always (also the decode layout's stand-in while its copy
                # cannot be built: under graph capture)
                ksplit = lib.g16_skinny_plan(M, N, K, _sm_count(dev))
                pl = PreparedCall(_clib.fast().skinny_f32in, "skinny GEMM")
                sizes = (lib.g16_skinny_workspace_bytes(M, N, K, ksplit),
                         lib.g16_skinny_counter_bytes(M, N, K, ksplit))
                if self.prepack_decode and lib.g16_skinny_strips_route(M, N, K, 1):
                    pls = PreparedCall(_clib.fast().skinny_strips_f32in, "skinny GEMM (decode layout)")
            entry = (pl, ksplit, sizes, w.data_ptr(), bptr, pls)
            self._skinny[key] = entry
        return entry

    def _weight_key(self) -> tuple:
        # what a copy of weight_t is valid for: its storage, in-place write counter and device
        w = self.weight_t
        return (w.data_ptr(), tensor_version(w), w.device)

    def _build_copy(self, old: torch.Tensor | None, pack) -> torch.Tensor:
        # Eager build of a copy of weight_t. Any stream may read a copy, so the device is synchronised
        # before the old copy is dropped (no kernel still reads it when the allocator reuses it) and
        # after the new one is written (complete before any stream reads it). Once per weight change.
        dev = self.weight_t.device
        if old is not None:
            torch.cuda.synchronize(old.device)
        new = pack(self.weight_t)
        torch.cuda.synchronize(dev)
        return new

    def _packed_weight(self) -> torch.Tensor | None:
        # the prepacked copy of weight_t, (re)built when weight_t is another tensor or was written in
        # place; None when it is not current and the stream is being captured (no build then)
        key = self._weight_key()
        if self._wp is None or self._wp_key != key:
            if torch.cuda.is_current_stream_capturing():
                return None
            self._wp = self._build_copy(self._wp, pack_weight)
            self._wp_key = key
        return self._wp

    def _decode_weight(self) -> int:
        # pointer of the decode-layout copy of weight_t, (re)built like the prepacked copy; 0 when it
        # is not current and the stream is being captured
        key = self._weight_key()
        if self._wd is None or self._wd_key != key:
            if torch.cuda.is_current_stream_capturing():
                return 0
            self._wd = self._build_copy(self._wd, pack_decode_weight)
            self._wd_key = key
            self._wd_ptr = self._wd.data_ptr()
        return self._wd_ptr

    def release_copies(self) -> None:
        """Free the prepacked and decode-layout copies of the weight (rebuilt on demand)."""
        if self._wp is not None or self._wd is not None:
            torch.cuda.synchronize(self.weight_t.device)
        self._wp = self._wd = None
        self._wp_key = self._wd_key = None
        self._wd_ptr = 0

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out_dtype = x.dtype if x.dtype in (torch.float32, torch.float16) else torch.float32
        if torch.is_grad_enabled() and x.requires_grad:
            return F.linear(x, self.weight_t.t().to(x.dtype), None if self.bias is None else self.bias.to(x.dtype))
        shape = x.shape
        # Fast path for small batches (generation): minimal Python per call (linear.py:49-64).
        # Unlike the reference, the weight's support is checked (once per layer and M), so a
        # FastLinear built directly with K or N not a multiple of 8 still takes the fallback.
        if x.is_cuda and x.dtype == torch.float32 and x.is_contiguous() and x.data_ptr() % 16 == 0:
            K, N = self.in_features, self.out_features
            M = x.numel() // K if shape[-1] == K else -1
            if 0 < M <= SKINNY_MAX_M:
                dev = x.device
                pl, ksplit, sizes, wptr, bptr, pls = self._decode_entry(M, dev)
                if pl is not None:
                    stream = stream_handle(dev.index or 0)
                    out = torch.empty(*shape[:-1], N, device=dev, dtype=torch.float32)
                    wd = 0
                    if pls is not None:
                        w = self.weight_t
                        wd = self._wd_ptr if self._wd_key == (wptr, tensor_version(w), w.device) else self._decode_weight()
                    if wd:
                        pls(x.data_ptr(), wd, out.data_ptr(), bptr, M, N, K, stream)
                    else:
                        bufs = split_buffers(dev, stream, *sizes)
                        pl(x.data_ptr(), wptr, out.data_ptr(), bptr, M, N, K, ksplit, *bufs, stream)
                    return out
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype not in (torch.float16, torch.float32):
            x2 = x2.float()
        # no cast to fp16 here: the library's rowscale pass does the cast, with the per-row scaling
        x2 = x2.contiguous()
        if x2.shape[0] == 0 or not supported(x2, self.weight_t):
            y = F.linear(x2.float(), self.weight_t.t().float(), None if self.bias is None else self.bias.float())
        else:
            odt = torch.float32 if out_dtype == torch.float32 else torch.float16
            M = x2.shape[0]
            b = self.bias
            wp = None
            if self.prepack_weight and M > SKINNY_MAX_M and \
                    prepacked_route(M, self.out_features, self.in_features, x2.device):
                wp = self._packed_weight()
            if wp is not None:
                y = mm_t_prepacked(x2, self.weight_t, wp, b, odt, _cast_source=x if self.share_cast else None)
            elif (self.prepack_decode and M <= STRIPS_MAX_M and x2.device == self.weight_t.device
                  and (b is None or (b.dtype == torch.float32 and b.device == x2.device))
                  and _clib.load().g16_skinny_strips_route(M, self.out_features, self.in_features,
                                                           int(x2.dtype == torch.float32))
                  and self._decode_weight()):
                # token-by-token calls the fast path above does not take (fp16 activations, views):
                # the decode layout where the library's rule expects a gain
                y = skinny_strips(x2, self._wd, b)
            else:
                y = mm_t(x2, self.weight_t, self.bias, odt)
        return y.reshape(*shape[:-1], self.out_features).to(out_dtype)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"


def patch(model: nn.Module, min_features: int = 256, force: bool = False, skip: tuple[str, ...] = ()) -> int:
    """Replace nn.Linear layers in place with FastLinear; returns the number replaced
    (linear.py:79-99).

    Runs only when a GPU parameter of the model is on a device these kernels target (gfx950), unless
    force=True. Layers on the GPU with in/out features >= min_features, both multiples of 8, and
    whose qualified name contains none of the strings in ``skip`` are replaced (e.g.
    skip=("lm_head",) keeps an output head in fp32).
    """
    if not force and not any(is_affected(p.device) for p in model.parameters() if p.is_cuda):
        return 0
    n = 0
    for name, mod in list(model.named_modules()):
        for child_name, child in list(mod.named_children()):
            full = f"{name}.{child_name}" if name else child_name
            if (isinstance(child, nn.Linear) and child.weight.is_cuda
                    and min(child.in_features, child.out_features) >= min_features
                    and child.in_features % 8 == 0 and child.out_features % 8 == 0
                    and not any(s in full for s in skip)):
                setattr(mod, child_name, FastLinear.from_linear(child))
                n += 1
    return n
