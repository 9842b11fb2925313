"""The functional op and the ``GatedDeltaNet2`` token mixer on the hip backend.

Mirrors the reference's ``gdn2/attention.py``: ``gdn2_attention`` (``:102-164``),
``resolve_backend`` (``:44-61``), ``GDN2Cache`` (``:172-183``) and the
``GatedDeltaNet2`` module (``:232-491``) with the same parameter names, so a
reference ``state_dict`` loads unchanged.

Backends: ``"auto"`` resolves to ``"hip"`` on a GPU and to ``"torch"``
elsewhere, like the reference's ``"tilelang"`` policy. ``"tilelang"``, the
reference's name for its GPU backend, is accepted and selects ``"hip"``, so a
reference config that names it explicitly runs the gfx950 kernels. The ``"torch"`` backend
is the reference package's own CPU path and is not part of this package, so it
raises ``NotImplementedError`` here. Autograd through ``gdn2_attention`` runs
the hip backward (``chunk_gdn2_bwd``).

Two layer details differ on purpose:

* ``init_cache`` keeps the recurrent state in ``dtype`` (fp32 by default) but
  allocates the short-conv tail in the conv weights' dtype, so a bf16 layer can
  decode (the reference allocates both in ``dtype`` and a bf16 layer's
  ``conv1d`` then fails on the mixed dtypes);
* the short-conv decode casts a cached tail to the activation dtype.

On a GPU the layer's work around the op runs as three launches besides the
op: one GEMM for all seven input projections (their weights concatenated once
and cached), ``gdn2_hip_layer_prologue`` (short conv + SiLU, L2 norm, gates,
decay, new conv tail) and ``gdn2_hip_layer_epilogue`` (gated RMSNorm); then
``o_proj``. CPU tensors take the torch formulas of the reference layer
(plumbing only: the op itself has no CPU path).
"""

from __future__ import annotations

import ctypes

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from . import _hip
from .config import DEFAULT_KERNEL_CONFIG, GDN2Config, GatedDeltaNet2Config
from .forward import check_cu_seqlens, chunk_gdn2_bwd, chunk_gdn2_fwd, chunk_gdn2_varlen_bwd, chunk_gdn2_varlen_fwd
from .inference import gdn2_decode, gdn2_prefill

__all__ = ["gdn2_attention", "GatedDeltaNet2", "GDN2Cache", "resolve_backend"]

_BACKENDS = ("auto", "hip", "tilelang", "torch")
# the reference's GPU backend name (gdn2/attention.py:41) selects this package's GPU path
_GPU_ALIASES = {"tilelang": "hip"}


def resolve_backend(backend: str, on_cuda: bool, needs_grad: bool) -> str:
    """Turn ``"auto"`` into a concrete backend, or validate an explicit one.

    Returns ``"hip"`` or ``"torch"``; raises ``ValueError`` for an unknown name
    or for a GPU backend (``"hip"``, or the reference's ``"tilelang"``, which
    maps to it) without a GPU, as the reference does for ``"tilelang"``
    (``gdn2/attention.py:44-61``).
    """
    if backend not in _BACKENDS:
        raise ValueError(f"unknown backend {backend!r}; expected one of {_BACKENDS}")
    if backend == "auto":
        return "hip" if on_cuda else "torch"
    if backend != "torch" and not on_cuda:
        raise ValueError(f"backend {backend!r} requires a CUDA device")
    return _GPU_ALIASES.get(backend, backend)


class _GDN2Function(torch.autograd.Function):
    """hip forward and backward (reference: ``gdn2/attention.py:60-99``)."""

    @staticmethod
    def forward(ctx, q, k, v, g, b, w, scale, initial_state, output_final_state, config):
        ctx.save_for_backward(q, k, v, g, b, w, initial_state)
        ctx.scale, ctx.config = scale, config
        return chunk_gdn2_fwd(q, k, v, g, b, w, scale, initial_state, output_final_state, config)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, do, dfinal_state):
        q, k, v, g, b, w, initial_state = ctx.saved_tensors
        if do is None:
            do = torch.zeros(*v.shape, dtype=q.dtype, device=q.device)
        dq, dk, dv, dg, db, dw, ds0 = chunk_gdn2_bwd(q, k, v, g, b, w, ctx.scale, initial_state, do, dfinal_state,
                                                     ctx.config)
        return dq, dk, dv, dg, db, dw, None, ds0, None, None


class _GDN2VarlenFunction(torch.autograd.Function):
    """Packed sequences: hip forward in one pass, hip backward per sequence."""

    @staticmethod
    def forward(ctx, q, k, v, g, b, w, scale, cu_seqlens, initial_state, output_final_state, config):
        ctx.save_for_backward(q, k, v, g, b, w, initial_state)
        ctx.scale, ctx.config, ctx.cu = scale, config, cu_seqlens
        return chunk_gdn2_varlen_fwd(q, k, v, g, b, w, scale, cu_seqlens, initial_state, output_final_state, config)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, do, dfinal_state):
        q, k, v, g, b, w, initial_state = ctx.saved_tensors
        if do is None:
            do = torch.zeros(*v.shape, dtype=q.dtype, device=q.device)
        dq, dk, dv, dg, db, dw, ds0 = chunk_gdn2_varlen_bwd(q, k, v, g, b, w, ctx.scale, ctx.cu, initial_state, do,
                                                            dfinal_state, ctx.config)
        return dq, dk, dv, dg, db, dw, None, None, ds0, None, None


def gdn2_attention(q, k, v, g, b, w, scale=None, initial_state=None, output_final_state=False,
                   config: GDN2Config = DEFAULT_KERNEL_CONFIG, cu_seqlens=None):
    """Gated DeltaNet-2 attention over a full sequence.

    Args:
        q, k: ``[B, S, H, DK]`` (the layer L2-normalises them); v: ``[B, S, H, DV]``.
        g: ``[B, S, H, DK]`` log decay (<= 0); b: ``[B, S, H, DK]`` erase gate;
        w: ``[B, S, H, DV]`` write gate.
        scale: query scale; defaults to ``DK ** -0.5``.
        initial_state: ``[B, H, DK, DV]`` or ``None``; never modified.
        output_final_state: also return the state after the last token.
        config: execution configuration.
        cu_seqlens: ``[N + 1]`` int offsets of N sequences packed in one batch
            row (B = 1); each runs its own recurrence, ``initial_state`` and
            the final state are then ``[N, H, DK, DV]``. The reference rejects
            packed batches (``gdn2/attention.py:142-145``); this backend runs
            them in one pass (the backward runs per sequence).

    Returns:
        ``(o [B, S, H, DV], final_state or None)``.
    """
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q, k, v, g, b, w, initial_state))
    backend = resolve_backend(config.backend, q.device.type == "cuda", needs_grad)
    if backend == "torch":
        raise NotImplementedError(
            "the 'torch' backend is the reference package's CPU path (gdn2.reference); "
            "this package provides the 'hip' backend only")
    if cu_seqlens is not None:
        if needs_grad:
            return _GDN2VarlenFunction.apply(q, k, v, g, b, w, scale, cu_seqlens, initial_state,
                                             output_final_state, config)
        return chunk_gdn2_varlen_fwd(q, k, v, g, b, w, scale, cu_seqlens, initial_state, output_final_state,
                                     config)
    if needs_grad:
        return _GDN2Function.apply(q, k, v, g, b, w, scale, initial_state, output_final_state, config)
    return chunk_gdn2_fwd(q, k, v, g, b, w, scale, initial_state, output_final_state, config)


# ---------------------------------------------------------------------------
# Module
# ---------------------------------------------------------------------------


@dataclass
class GDN2Cache:
    """Per-layer decoding cache.

    Attributes:
        recurrent_state: ``[B, H_v, DK, DV]`` fp32 carried state.
        conv_state: ``[B, C, conv_size - 1]`` tail of the short-conv input, or
            ``None`` when the layer has no short convolution.
    """

    recurrent_state: torch.Tensor
    conv_state: torch.Tensor | None = None


class _ShortConv(nn.Module):
    """Causal depthwise conv1d + SiLU over ``[B, S, C]``, with a decode tail."""

    def __init__(self, channels: int, kernel_size: int = 4, activation: bool = True):
        super().__init__()
        self.channels = channels
        self.kernel_size = kernel_size
        self.activation = activation
        self.conv = nn.Conv1d(channels, channels, kernel_size, groups=channels, padding=kernel_size - 1)

    def _act(self, y):
        return F.silu(y) if self.activation else y

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self.conv(x.transpose(1, 2))[..., : x.shape[1]]
        return self._act(y.transpose(1, 2))

    def step(self, x: torch.Tensor, state: torch.Tensor):
        y, state = self.decode(x.unsqueeze(1), state)
        return y[:, 0], state

    def decode(self, x: torch.Tensor, state: torch.Tensor):
        """``x [B, n, C]`` continuing from the cached ``kernel_size - 1`` inputs."""
        buf = torch.cat([state.to(x.dtype), x.transpose(1, 2)], dim=-1)
        y = F.conv1d(buf, self.conv.weight, self.conv.bias, groups=self.channels)
        return self._act(y.transpose(1, 2)), buf[..., buf.shape[-1] - (self.kernel_size - 1):]


class _GatedRMSNorm(nn.Module):
    """Per-head RMSNorm followed by a SiLU output gate."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (xf * self.weight * F.silu(gate.float())).to(gate.dtype)


class GatedDeltaNet2(nn.Module):
    """Gated DeltaNet-2 token mixer with a serving cache.

    The erase gate ``b`` lives on the key axis, the write gate ``w`` on the
    value axis; decay ``g = -exp(A_log) * softplus(f + dt_bias)`` is per key
    channel. Key heads are repeated up to ``num_heads`` value heads.
    """

    def __init__(self, config: GatedDeltaNet2Config):
        super().__init__()
        self.cfg = config
        H = config.num_heads
        HK = config.num_kv_heads or H
        if H % HK:
            raise ValueError(f"num_heads {H} must be a multiple of num_kv_heads {HK}")
        DK = config.head_dim_k
        DV = config.head_dim_v or DK
        self.num_heads, self.num_kv_heads = H, HK
        self.head_dim_k, self.head_dim_v = DK, DV
        self.head_repeat = H // HK
        d_qk, d_v, hid = HK * DK, H * DV, config.hidden_size

        self.q_proj = nn.Linear(hid, d_qk, bias=False)
        self.k_proj = nn.Linear(hid, d_qk, bias=False)
        self.v_proj = nn.Linear(hid, d_v, bias=False)
        self.b_proj = nn.Linear(hid, d_qk, bias=False)
        self.w_proj = nn.Linear(hid, d_v, bias=False)
        self.f_proj = nn.Linear(hid, d_qk, bias=False)
        self.o_gate_proj = nn.Linear(hid, d_v, bias=False)
        self.o_proj = nn.Linear(d_v, hid, bias=False)
        if config.conv_size > 0:
            self.q_conv = _ShortConv(d_qk, config.conv_size)
            self.k_conv = _ShortConv(d_qk, config.conv_size)
            self.v_conv = _ShortConv(d_v, config.conv_size)
        else:
            self.q_conv = self.k_conv = self.v_conv = None

        lo, hi = config.a_init_range
        self.A_log = nn.Parameter(torch.empty(HK).uniform_(lo, hi).log_())
        dt_lo, dt_hi = config.dt_init_range
        dt = torch.empty(HK, DK).uniform_(dt_lo, dt_hi)
        # softplus^-1(dt) so the initial step is exactly dt
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        self.o_norm = _GatedRMSNorm(DV, config.norm_eps)
        self.scale = DK ** -0.5
        self.erase_scale = config.erase_gate_scale

    # -- fused GPU path ------------------------------------------------------
    def _cat_cached(self, name, parts):
        """torch.cat(parts) along dim 0, rebuilt only when a part changes
        (tracked by storage pointer and version counter)."""
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in parts)
        hit = self.__dict__.get(name)
        if hit is None or hit[0] != key:
            hit = (key, torch.cat([t.detach().reshape(t.shape[0], -1) for t in parts], 0).contiguous())
            self.__dict__[name] = hit
        return hit[1]

    def _f32_cached(self, name, t):
        """Contiguous fp32 copy of parameter ``t``, rebuilt only when it changes."""
        key = (t.data_ptr(), t._version, t.dtype, t.device)
        hit = self.__dict__.get(name)
        if hit is None or hit[0] != key:
            hit = (key, t.detach().float().contiguous())
            self.__dict__[name] = hit
        return hit[1]

    def _linear(self, x2, weight):
        """x2 [M, K] @ weight^T. A few rows (decode) go through the library's
        GEMV, which streams the weight once; more rows through torch."""
        M, K = x2.shape
        if (1 <= M <= 8 and K % 8 == 0 and x2.dtype == weight.dtype and weight.is_contiguous()
                and not (torch.is_grad_enabled() and (weight.requires_grad or x2.requires_grad))
                and x2.stride(1) == 1 and x2.stride(0) % 8 == 0 and x2.data_ptr() % 16 == 0
                and weight.data_ptr() % 16 == 0):
            y = torch.empty(M, weight.shape[0], device=x2.device, dtype=x2.dtype)
            _hip.check(_hip.lib().gdn2_hip_gemv(
                x2.data_ptr(), x2.stride(0), weight.data_ptr(), y.data_ptr(), y.stride(0),
                _hip.dtype_code(x2.dtype), M, weight.shape[0], K, _hip.stream_of(x2.device)), "gdn2_hip_gemv")
            return y
        return F.linear(x2, weight)

    def _proj_weights(self):
        # one [4*HK*DK + 3*H*DV, hidden] weight: q | k | v | b | w | f | o_gate
        return self._cat_cached("_wcat", [self.q_proj.weight, self.k_proj.weight, self.v_proj.weight,
                                          self.b_proj.weight, self.w_proj.weight, self.f_proj.weight,
                                          self.o_gate_proj.weight])

    def _project_gpu(self, x, cache, conv_tail=False, cu=None):
        """All projections in one GEMM, then the prologue kernel. Returns the op
        inputs, the projection buffer (its o_gate columns feed _finish_gpu) and
        the new conv tail (or None). ``cu``: int32 device offsets of N packed
        sequences (B = 1): each token's conv window starts at its own
        sequence's first token, continuing from that sequence's cached tail
        (``cache.conv_state`` [N, C, K-1]); the new tails are [N, C, K-1]."""
        B, S, hid = x.shape
        HK, H, DK, DV = self.num_kv_heads, self.num_heads, self.head_dim_k, self.head_dim_v
        dqk, dv = HK * DK, H * DV
        dt = x.dtype
        proj = self._linear(x.reshape(B * S, hid), self._proj_weights())     # [B*S, 4 dqk + 3 dv]
        ld = proj.shape[1]
        es = proj.element_size()
        base = proj.data_ptr()
        offs = [0, dqk, 2 * dqk, 2 * dqk + dv, 3 * dqk + dv, 3 * dqk + 2 * dv]   # q k v b w f
        dev = x.device
        q = torch.empty(B, S, HK, DK, device=dev, dtype=dt)
        k = torch.empty_like(q)
        b = torch.empty_like(q)
        v = torch.empty(B, S, H, DV, device=dev, dtype=dt)
        w = torch.empty_like(v)
        g = torch.empty(B, S, HK, DK, device=dev, dtype=torch.float32)
        conv_w = conv_b = conv_in = conv_out = None
        K = 0
        if self.q_conv is not None:
            K = self.cfg.conv_size
            convs = (self.q_conv.conv, self.k_conv.conv, self.v_conv.conv)
            conv_w = self._cat_cached("_convw", [c.weight for c in convs])
            if conv_w.dtype != dt:
                conv_w = conv_w.to(dt)
            if all(c.bias is not None for c in convs):
                conv_b = self._cat_cached("_convb", [c.bias for c in convs])
                conv_b = conv_b.to(dt).reshape(-1) if conv_b.dtype != dt else conv_b.reshape(-1)
            if cache is not None and cache.conv_state is not None:
                conv_in = cache.conv_state.to(dt).contiguous()
                if conv_in.data_ptr() % 16:          # the kernel reads 16-byte vectors
                    conv_in = conv_in.clone()
            if cache is not None or conv_tail:
                nrow = B if cu is None else cu.numel() - 1
                conv_out = torch.empty(nrow, 2 * dqk + dv, K - 1, device=dev, dtype=dt)
        a_log = self._f32_cached("_alog32", self.A_log)
        dt_bias = self._f32_cached("_dtb32", self.dt_bias)
        P = _hip.ptr
        if cu is not None:
            _hip.check(_hip.lib().gdn2_hip_layer_prologue_varlen(
                *(base + o * es for o in offs), ld, ld, ld, ld, ld, ld, _hip.dtype_code(dt),
                P(conv_w), P(conv_b), K, P(conv_in), P(conv_out), P(a_log), P(dt_bias), float(self.erase_scale),
                P(q), P(k), P(v), P(b), P(w), P(g), P(cu), cu.numel() - 1, S, H, HK, DK, DV,
                _hip.stream_of(dev)), "gdn2_hip_layer_prologue_varlen")
            return (q, k, v, g, b, w), proj, conv_out
        _hip.check(_hip.lib().gdn2_hip_layer_prologue(
            *(base + o * es for o in offs), ld, ld, ld, ld, ld, ld, _hip.dtype_code(dt),
            P(conv_w), P(conv_b), K, P(conv_in), P(conv_out), P(a_log), P(dt_bias), float(self.erase_scale),
            P(q), P(k), P(v), P(b), P(w), P(g), B, S, H, HK, DK, DV, _hip.stream_of(dev)),
            "gdn2_hip_layer_prologue")
        return (q, k, v, g, b, w), proj, conv_out

    def _finish_gpu(self, x, o, proj):
        B, S, _ = x.shape
        if B * S == 0:
            return x.new_empty(B, S, self.cfg.hidden_size)
        H, DV = self.num_heads, self.head_dim_v
        dqk, dv = self.num_kv_heads * self.head_dim_k, H * DV
        ld = proj.shape[1]
        gate_ptr = proj.data_ptr() + (4 * dqk + 2 * dv) * proj.element_size()
        out = torch.empty(B, S, dv, device=x.device, dtype=x.dtype)
        o = o.contiguous()
        weight = self._f32_cached("_onw32", self.o_norm.weight)
        _hip.check(_hip.lib().gdn2_hip_layer_epilogue(
            _hip.ptr(o), _hip.dtype_code(o.dtype), gate_ptr, ld, _hip.ptr(weight), float(self.o_norm.eps),
            _hip.ptr(out), _hip.dtype_code(x.dtype), dv, B, S, H, DV, _hip.stream_of(x.device)),
            "gdn2_hip_layer_epilogue")
        return self._linear(out.reshape(B * S, dv), self.o_proj.weight).view(B, S, -1)

    def _decode_params(self):
        """The parameters the fused decode reads, looked up through the module
        dicts (not nn.Module attribute access, which costs ~0.3 us a lookup)."""
        m = self._modules
        ps = [m[n]._parameters["weight"] for n in ("q_proj", "k_proj", "v_proj", "b_proj", "w_proj", "f_proj",
                                                    "o_gate_proj", "o_proj")]
        if m.get("q_conv") is not None:
            for n in ("q_conv", "k_conv", "v_conv"):
                cp = m[n]._modules["conv"]._parameters
                ps.append(cp["weight"])
                ps.append(cp["bias"])
        ps.append(self._parameters["A_log"])
        ps.append(self._parameters["dt_bias"])
        ps.append(m["o_norm"]._parameters["weight"])
        return ps

    def _decode_plan(self, B, n, dt, device):
        """The static part of a fused decode call for (B, n, dtype, device): the
        cached weight buffers and the C-ABI arguments that do not change between
        calls, rebuilt when any parameter is replaced or changed in place.
        None when the shapes do not qualify."""
        ps = self._decode_params()
        key = (B, n, dt, device, tuple(map(id, ps)), tuple(t._version for t in ps))
        hit = self.__dict__.get("_dec_plan")
        if hit is not None and hit[0] == key:
            return hit[1]
        HK, H, DK, DV = self.num_kv_heads, self.num_heads, self.head_dim_k, self.head_dim_v
        hid = self.cfg.hidden_size
        plan = None
        if not (B * n > 8 or hid % 8 or (H * DV) % 8 or DK % 8 or (DK // 8) & (DK // 8 - 1) or DK > 512
                or DV % 32 or DK not in (32, 64, 128, 256) or self.o_proj.weight.dtype != dt):
            w_out = self.o_proj.weight.detach()
            if w_out.is_contiguous():
                lib = _hip.lib()
                code = _hip.dtype_code(dt)
                ws = torch.empty(lib.gdn2_hip_layer_decode_workspace_bytes(B, n, H, HK, DK, DV, code) + 256,
                                 dtype=torch.uint8, device=device)
                w_proj = self._proj_weights()
                conv_w = conv_b = None
                K = 0
                if self.q_conv is not None:
                    K = self.cfg.conv_size
                    convs = (self.q_conv.conv, self.k_conv.conv, self.v_conv.conv)
                    conv_w = self._cat_cached("_convw", [c.weight for c in convs])
                    if conv_w.dtype != dt:
                        conv_w = conv_w.to(dt)
                    if all(c.bias is not None for c in convs):
                        conv_b = self._cat_cached("_convb", [c.bias for c in convs])
                        conv_b = conv_b.to(dt).reshape(-1) if conv_b.dtype != dt else conv_b.reshape(-1)
                alog = self._f32_cached("_alog32", self.A_log)
                dtb = self._f32_cached("_dtb32", self.dt_bias)
                onw = self._f32_cached("_onw32", self.o_norm.weight)
                P = _hip.ptr
                ws_ptr = (ws.data_ptr() + 255) // 256 * 256
                plan = dict(
                    # the parameters are held too, so the ids in the key stay theirs
                    keep=(ws, w_proj, conv_w, conv_b, alog, dtb, onw, w_out, ps), K=K,
                    C=2 * HK * DK + H * DV, fn=lib.gdn2_hip_layer_decode,
                    # arguments between x and conv_in, conv_out and the state, the state and
                    # out, and after out (gdn2_hip_layer_decode's order)
                    a1=(P(w_proj), P(conv_w), P(conv_b), K),
                    a2=(P(alog), P(dtb), float(self.erase_scale)),
                    a3=(P(onw), float(self.o_norm.eps), P(w_out)),
                    a4=(ctypes.c_void_p(ws_ptr), code, B, n, hid, H, HK, DK, DV, float(self.scale)))
        self.__dict__["_dec_plan"] = (key, plan)
        return plan

    def _decode_fused(self, x, cache):
        """A decode call of B*n <= 8 tokens as one library call
        (gdn2_hip_layer_decode: projections, prologue, recurrence, gated norm,
        o_proj). Returns the output, or None when the shapes or the cache do not
        qualify (the caller then takes the per-stage path)."""
        B, n, hid = x.shape
        st = cache.recurrent_state
        dt = x.dtype
        if (st is None or st.dtype != torch.float32 or not st.is_contiguous() or st.device != x.device
                or tuple(st.shape) != (B, self.num_heads, self.head_dim_k, self.head_dim_v)):
            return None
        plan = self._decode_plan(B, n, dt, x.device)
        if plan is None:
            return None
        x2 = x.reshape(B * n, hid)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        if x2.data_ptr() % 16:
            x2 = x2.clone()
        conv_in = conv_out = None
        K = plan["K"]
        if K:
            conv_in = cache.conv_state
            if conv_in is not None and (conv_in.dtype != dt or not conv_in.is_contiguous()
                                        or conv_in.data_ptr() % 16):
                conv_in = conv_in.to(dt).contiguous()
                if conv_in.data_ptr() % 16:
                    conv_in = conv_in.clone()
            conv_out = torch.empty(B, plan["C"], K - 1, device=x.device, dtype=dt)
        out = torch.empty(B, n, hid, device=x.device, dtype=dt)
        P = _hip.ptr
        _hip.check(plan["fn"](P(x2), *plan["a1"], P(conv_in), P(conv_out), *plan["a2"], st.data_ptr(),
                              *plan["a3"], out.data_ptr(), *plan["a4"], _hip.stream_of(x.device)),
                   "gdn2_hip_layer_decode")
        if K:
            cache.conv_state = conv_out
        return out

    # -- pieces shared by forward / prefill / decode -----------------------
    def _decay(self, x, lead):
        f = self.f_proj(x).view(*lead, self.num_kv_heads, self.head_dim_k)
        return -self.A_log.exp().unsqueeze(-1) * F.softplus(f.float() + self.dt_bias)

    def _conv_with_cache(self, q, k, v, cache):
        if self.q_conv is None:
            return q, k, v
        d = self.num_kv_heads * self.head_dim_k
        cs = cache.conv_state
        q, cq = self.q_conv.decode(q, cs[:, :d])
        k, ck = self.k_conv.decode(k, cs[:, d:2 * d])
        v, cv = self.v_conv.decode(v, cs[:, 2 * d:])
        cache.conv_state = torch.cat([cq, ck, cv], dim=1)
        return q, k, v

    def _project(self, x, cache):
        """Projections, short conv, L2 norm and gates -> op inputs.

        q, k, b, g stay on the HK key heads: the hip op reads key head
        h // (H // HK) for value head h, which is what the reference's
        ``repeat_interleave`` (``attention.py:295-297``) computes, without
        materialising the repeated tensors.
        """
        B, S, _ = x.shape
        HK, H, DK, DV = self.num_kv_heads, self.num_heads, self.head_dim_k, self.head_dim_v
        q, k, v = self.q_proj(x), self.k_proj(x), self.v_proj(x)
        if cache is not None:
            q, k, v = self._conv_with_cache(q, k, v, cache)
        elif self.q_conv is not None:
            q, k, v = self.q_conv(q), self.k_conv(k), self.v_conv(v)
        q = F.normalize(q.view(B, S, HK, DK), p=2, dim=-1)
        k = F.normalize(k.view(B, S, HK, DK), p=2, dim=-1)
        v = v.view(B, S, H, DV)
        g = self._decay(x, (B, S))
        b = torch.sigmoid(self.b_proj(x).view(B, S, HK, DK)) * self.erase_scale
        w = torch.sigmoid(self.w_proj(x).view(B, S, H, DV))
        return q.contiguous(), k.contiguous(), v.contiguous(), g.contiguous(), b.contiguous(), w.contiguous()

    def _finish(self, x, o):
        B, S, _ = x.shape
        gate = self.o_gate_proj(x).view(B, S, self.num_heads, self.head_dim_v)
        return self.o_proj(self.o_norm(o, gate).reshape(B, S, -1))

    # -- public API ---------------------------------------------------------
    def forward(self, hidden_states, cache=None, use_cache=False, cu_seqlens=None):
        """Full-sequence mixer (training form). Returns ``(output, cache or None)``."""
        B, S, _ = hidden_states.shape
        if cu_seqlens is not None and hidden_states.is_cuda:
            if torch.is_grad_enabled() and (hidden_states.requires_grad or
                                            any(p.requires_grad for p in self.parameters())):
                raise NotImplementedError("training GatedDeltaNet2 on packed sequences (cu_seqlens) is not "
                                          "provided; gdn2_attention(cu_seqlens=...) itself is differentiable")
            # packed sequences: per-sequence conv windows in the prologue and the
            # packed op; as for a dense batch, the conv starts fresh (the
            # cache's conv tails are not read) and the recurrent state carries on
            if B != 1:
                raise ValueError(f"packed sequences (cu_seqlens) need batch size 1; got {B}")
            cu = check_cu_seqlens(cu_seqlens, S).to(hidden_states.device)
            N = cu.numel() - 1
            if cache is not None and cache.recurrent_state.shape[0] != N:
                raise ValueError(f"a packed batch of {N} sequences needs a cache of {N} rows; "
                                 f"got {cache.recurrent_state.shape[0]}")
            (q, k, v, g, b, w), proj, conv_state = self._project_gpu(hidden_states, None, conv_tail=use_cache,
                                                                     cu=cu)
            o, final_state = gdn2_attention(
                q, k, v, g, b, w, scale=self.scale,
                initial_state=cache.recurrent_state if cache is not None else None,
                output_final_state=use_cache, config=self.cfg.kernel, cu_seqlens=cu)
            out = self._finish_gpu(hidden_states, o, proj)
            return out, (GDN2Cache(final_state, conv_state) if use_cache else None)
        if cu_seqlens is not None and self.q_conv is not None:
            raise NotImplementedError("packed sequences (cu_seqlens) through the layer's short convolution "
                                      "run on the GPU only")
        if hidden_states.is_cuda and S == 0:             # nothing to run: the state carries over
            return self._empty_call(hidden_states, cache, use_cache, fresh_conv=True)
        # training: the projections, conv, gates and norm as torch ops (autograd),
        # the attention op through gdn2_attention's hip forward and backward
        trains = torch.is_grad_enabled() and (hidden_states.requires_grad or
                                              any(p.requires_grad for p in self.parameters()))
        if hidden_states.is_cuda and not trains:
            (q, k, v, g, b, w), proj, conv_state = self._project_gpu(hidden_states, None, conv_tail=use_cache)
            o, final_state = gdn2_attention(
                q, k, v, g, b, w, scale=self.scale,
                initial_state=cache.recurrent_state if cache is not None else None,
                output_final_state=use_cache, config=self.cfg.kernel, cu_seqlens=cu_seqlens)
            out = self._finish_gpu(hidden_states, o, proj)
            return out, (GDN2Cache(final_state, conv_state) if use_cache else None)
        conv_state = None
        if self.q_conv is not None and use_cache:
            width = self.cfg.conv_size - 1
            raw = torch.cat([self.q_proj(hidden_states), self.k_proj(hidden_states),
                             self.v_proj(hidden_states)], dim=-1).transpose(1, 2)
            padded = F.pad(raw, (max(0, width - S), 0))
            conv_state = padded[..., padded.shape[-1] - width:]
        q, k, v, g, b, w = self._project(hidden_states, None)
        o, final_state = gdn2_attention(
            q, k, v, g, b, w, scale=self.scale,
            initial_state=cache.recurrent_state if cache is not None else None,
            output_final_state=use_cache, config=self.cfg.kernel, cu_seqlens=cu_seqlens)
        out = self._finish(hidden_states, o)
        return out, (GDN2Cache(final_state, conv_state) if use_cache else None)

    @torch.no_grad()
    def prefill(self, hidden_states, cache=None, *, cu_seqlens=None):
        """Prefill a prompt (or one segment of it); returns ``(output, cache)``.

        ``cu_seqlens`` (an extension; GPU only): ``hidden_states`` is ``[1, T,
        hidden]`` holding N packed prompts, and the cache (``None``: fresh)
        has N rows; each sequence continues from its own recurrent state and
        conv tail, and the returned cache has one of each per sequence."""
        if cu_seqlens is not None:
            return self._prefill_packed(hidden_states, cache, cu_seqlens)
        if cache is None:
            cache = self.init_cache(hidden_states.shape[0], device=hidden_states.device)
        if hidden_states.is_cuda and hidden_states.shape[1] == 0:
            return self._empty_call(hidden_states, cache, True, fresh_conv=False)
        if hidden_states.is_cuda:
            (q, k, v, g, b, w), proj, conv_out = self._project_gpu(hidden_states, cache)
            cache.conv_state = conv_out
            o, state = gdn2_prefill(q, k, v, g, b, w, cache.recurrent_state, scale=self.scale,
                                    config=self.cfg.kernel)
            cache.recurrent_state = state
            return self._finish_gpu(hidden_states, o, proj), cache
        q, k, v, g, b, w = self._project(hidden_states, cache)
        o, state = gdn2_prefill(q, k, v, g, b, w, cache.recurrent_state, scale=self.scale,
                                config=self.cfg.kernel)
        cache.recurrent_state = state
        return self._finish(hidden_states, o), cache

    def _empty_call(self, x, cache, use_cache, fresh_conv):
        """A call of zero tokens: empty output; the recurrent state carries over
        and the conv tail is zeros (forward: a fresh conv) or the cached one."""
        B = x.shape[0]
        out = x.new_empty(B, 0, self.cfg.hidden_size)
        if not use_cache:
            return out, None
        state = (cache.recurrent_state.clone() if cache is not None
                 else self.init_cache(B, device=x.device).recurrent_state)
        conv = None
        if self.q_conv is not None:
            C = 2 * self.num_kv_heads * self.head_dim_k + self.num_heads * self.head_dim_v
            if fresh_conv or cache is None or cache.conv_state is None:
                conv = torch.zeros(B, C, self.cfg.conv_size - 1, device=x.device, dtype=x.dtype)
            else:
                conv = cache.conv_state
        return out, GDN2Cache(state, conv)

    def _prefill_packed(self, x, cache, cu_seqlens):
        if not x.is_cuda:
            raise ValueError("packed prefill (cu_seqlens) requires a CUDA device (a ROCm GPU)")
        B, S, _ = x.shape
        if B != 1:
            raise ValueError(f"packed sequences (cu_seqlens) need batch size 1; got {B}")
        cu = check_cu_seqlens(cu_seqlens, S).to(x.device)
        N = cu.numel() - 1
        if cache is None:
            cache = self.init_cache(N, device=x.device)
        elif cache.recurrent_state.shape[0] != N:
            raise ValueError(f"a packed batch of {N} sequences needs a cache of {N} rows; "
                             f"got {cache.recurrent_state.shape[0]}")
        (q, k, v, g, b, w), proj, conv_out = self._project_gpu(x, cache, cu=cu)
        o, state = gdn2_attention(q, k, v, g, b, w, scale=self.scale, initial_state=cache.recurrent_state,
                                  output_final_state=True, config=self.cfg.kernel, cu_seqlens=cu)
        return self._finish_gpu(x, o, proj), GDN2Cache(state, conv_out)

    @torch.no_grad()
    def decode(self, hidden_states, cache):
        """Decode ``n`` tokens ``[B, n, hidden]``, updating ``cache`` in place."""
        return self._decode(hidden_states, cache)

    def _decode(self, hidden_states, cache):
        if hidden_states.is_cuda:
            out = self._decode_fused(hidden_states, cache)
            if out is not None:
                return out, cache
            (q, k, v, g, b, w), proj, conv_out = self._project_gpu(hidden_states, cache)
            cache.conv_state = conv_out
            o = gdn2_decode(q, k, v, g, b, w, cache.recurrent_state, scale=self.scale)
            return self._finish_gpu(hidden_states, o, proj), cache
        q, k, v, g, b, w = self._project(hidden_states, cache)
        o = gdn2_decode(q, k, v, g, b, w, cache.recurrent_state, scale=self.scale)
        return self._finish(hidden_states, o), cache

    @torch.no_grad()
    def step(self, hidden_states, cache):
        """Decode one token ``[B, hidden]``."""
        out, cache = self._decode(hidden_states.unsqueeze(1), cache)
        return out[:, 0], cache

    def init_cache(self, batch_size, device=None, dtype=torch.float32):
        """Empty cache: zero recurrent state in ``dtype``, zero conv tail in the
        conv weights' dtype."""
        state = torch.zeros(batch_size, self.num_heads, self.head_dim_k, self.head_dim_v,
                            device=device, dtype=dtype)
        conv_state = None
        if self.q_conv is not None:
            C = 2 * self.num_kv_heads * self.head_dim_k + self.num_heads * self.head_dim_v
            conv_state = torch.zeros(batch_size, C, self.cfg.conv_size - 1, device=device,
                                     dtype=self.q_conv.conv.weight.dtype)
        return GDN2Cache(state, conv_state)
