"""OrthoLinear: the dual-manifold linear layer, on MI355X.

API-compatible with /root/reference/torch_bind/ortho_linear.py:30-168:

  OrthoLinear(in_features, out_features, q_bits=4, bias=False, device=None, dtype=None)
  .set_alpha(alpha)                                   the privacy kill switch
  .load_from_weights(base_weight, ortho_weight, base_scales=None)
  .forward(x)                                         y = Base(x) + alpha*Ortho(x) (+ bias)

with the same buffers, names, dtypes and shapes, so a reference
``state_dict`` loads unchanged:

  base_weight        uint8  [out, in/2]  packed signed INT4, low nibble = even k
  base_scales        fp16   [out]        (or [out, in/G] with the group extension)
  ortho_values       fp16   [nnz]
  ortho_col_indices  int32  [nnz]
  ortho_row_ptr      int32  [out+1]      (empty until weights are loaded)

Differences, all deliberate:
  * ``group_size`` (keyword, default None = per-row scales as in the
    reference) selects FP16 scales per group of G input columns.
  * ``device`` is honoured for the buffers (the reference ignores it).
  * ``forward`` on a CPU tensor raises instead of returning uninitialised
    memory (the reference's CPU branch is ``pass``, :152-162); there is no
    CPU path in this library.
  * The ortho plan read by the kernels (a derived layout of the CSR
    buffers) is built on the first call with alpha > 0 and cached; it is
    rebuilt whenever one of the three CSR buffers is replaced or modified in
    place.  It is not a buffer and is not saved in the state_dict.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .. import _C_ops as _C
from .. import _lib
from ..tools.sieve import pack_ortho_sparse

HAS_C_OPS = True  # the reference's flag (:15-28); this package has no fallback


def load_checkpoint(model: nn.Module, path, map_location=None, strict: bool = True):
    """Loads a ``torch.save``d state_dict (from this package or from the
    reference's OrthoLinear modules) into ``model``.  The file is read with
    ``weights_only=True``: tensors and plain containers only, nothing in it
    is executed."""
    sd = torch.load(path, map_location=map_location, weights_only=True)
    if isinstance(sd, dict) and "state_dict" in sd and isinstance(sd["state_dict"], dict):
        sd = sd["state_dict"]
    return model.load_state_dict(sd, strict=strict)


def pack_base_torch(base_weight: torch.Tensor, group_size: Optional[int] = None,
                    base_scales: Optional[torch.Tensor] = None):
    """The torch-op form of the Base packing of load_from_weights
    (/root/reference/torch_bind/ortho_linear.py:89-120, plus group scales):
    (q uint8 [N, K/2], scales float16 [N] or [N, K/G]) on base_weight's device."""
    N, K = base_weight.shape
    G = K if group_size is None else group_size
    if base_scales is None:
        grouped = base_weight.reshape(N, K // G, G)
        scales = (grouped.abs().amax(dim=2) / 7.0).clamp(min=1e-6)
        if group_size is None:
            scales = scales.reshape(N)
    else:
        scales = base_scales
    s_full = scales.reshape(N, -1).to(base_weight.device)
    s_full = s_full.repeat_interleave(K // s_full.shape[1], dim=1)
    w_int = (base_weight / s_full).round().clamp(-8, 7).to(torch.int8)
    w_flat = w_int.flatten()
    packed = (w_flat[0::2] & 0x0F) | ((w_flat[1::2] & 0x0F) << 4)
    return packed.to(torch.uint8).view(N, -1), scales.to(dtype=torch.float16)


class OrthoLinear(nn.Module):
    """Y = X @ W_base^T + alpha * (X @ W_ortho^T) (+ bias)."""

    def __init__(self, in_features: int, out_features: int, q_bits: int = 4, bias: bool = False,
                 device=None, dtype=None, group_size: Optional[int] = None):
        super().__init__()
        if q_bits != 4:
            raise ValueError("OrthoLinear supports q_bits=4 only")
        if in_features % 2 != 0:
            raise ValueError("in_features must be even (two INT4 weights per byte)")
        if group_size is not None and (group_size <= 0 or in_features % group_size != 0):
            raise ValueError(f"group_size {group_size} must divide in_features {in_features}")
        self.in_features = in_features
        self.out_features = out_features
        self.q_bits = q_bits
        self.group_size = group_size
        scale_shape = (out_features,) if group_size is None else (out_features, in_features // group_size)
        self.register_buffer("base_weight", torch.zeros(out_features, in_features // 2,
                                                        dtype=torch.uint8, device=device))
        self.register_buffer("base_scales", torch.zeros(scale_shape, dtype=torch.float16, device=device))
        self.register_buffer("ortho_values", torch.tensor([], dtype=torch.float16, device=device))
        self.register_buffer("ortho_col_indices", torch.tensor([], dtype=torch.int32, device=device))
        self.register_buffer("ortho_row_ptr", torch.tensor([], dtype=torch.int32, device=device))
        self.alpha = 1.0
        if bias:
            self.register_parameter("bias", nn.Parameter(
                torch.zeros(out_features, dtype=dtype or torch.float32, device=device)))
        else:
            self.register_parameter("bias", None)
        self._plan = None
        self._plan_key = None
        self._plan_fast = None

    def set_alpha(self, alpha: float):
        """The kill switch: the ortho term is applied iff alpha > 0."""
        self.alpha = alpha

    @torch.no_grad()
    def load_from_weights(self, base_weight: torch.Tensor, ortho_weight: torch.Tensor,
                          base_scales: Optional[torch.Tensor] = None):
        """Quantise ``base_weight`` to INT4 and pack ``ortho_weight`` as CSR.

        Follows /root/reference/torch_bind/ortho_linear.py:79-128: scales =
        clamp(max|W| / 7, min=1e-6) per output row unless given; the FP16
        copy is stored, but q = clamp(round(W / scales), -8, 7) uses the
        scales as given; nibble pairs packed low = even index.  With
        ``group_size`` the max is taken per group and ``base_scales`` may be
        given as [out, in/G].
        """
        device = ortho_weight.device
        N, K = self.out_features, self.in_features
        if tuple(base_weight.shape) != (N, K) or tuple(ortho_weight.shape) != (N, K):
            raise ValueError(f"weights must be [{N}, {K}]")
        if base_weight.is_cuda and base_weight.dtype in (torch.float16, torch.bfloat16, torch.float32) and \
                (base_scales is None or base_scales.device == base_weight.device):
            # the library's packing kernels: the same bits as the torch ops below
            q, scales16 = _C.pack_base(base_weight, self.group_size, base_scales)
        else:
            q, scales16 = pack_base_torch(base_weight, self.group_size, base_scales)
        self.base_scales.data = scales16.to(device)
        self.base_weight.data = q.to(device)

        row_ptr, col_indices, values = pack_ortho_sparse(ortho_weight, format="csr")
        self.ortho_row_ptr = row_ptr.to(device=device, dtype=torch.int32)
        self.ortho_col_indices = col_indices.to(device=device, dtype=torch.int32)
        self.ortho_values = values.to(device=device, dtype=torch.float16)
        self._plan = None
        self._plan_key = None
        self._plan_fast = None

    # ------------------------------------------------------------------ plan
    def _csr_key(self):
        # the tensors themselves (compared by identity, kept alive by the key,
        # so a new tensor reusing a freed block is never taken for the old
        # one) and their versions (in-place writes)
        ts = (self.ortho_values, self.ortho_col_indices, self.ortho_row_ptr)
        return ts, tuple((t._version, t.data_ptr(), t.numel()) for t in ts)

    def _plan_valid(self, key) -> bool:
        if self._plan_key is None:
            return False
        (ts0, v0), (ts1, v1) = self._plan_key, key
        return all(a is b for a, b in zip(ts0, ts1)) and v0 == v1

    def _ortho_plan(self):
        """The cached ortho plan, rebuilt when the CSR buffers change.  A
        stream other than the one that built it waits on the build once, and
        the plan's memory is recorded on it (so a rebuilt plan's old memory
        is not reused before that stream's work is done).  Under graph
        capture a valid plan is used as is (torch.cuda.graph synchronises
        the device before capturing); a missing or stale one is not built
        there (building reads the plan's flags back, a synchronisation a
        capture does not allow): the captured call reads the CSR instead."""
        if self.ortho_values.numel() == 0 or not self.ortho_values.is_cuda:
            return None
        key = self._csr_key()
        dev = self.ortho_values.get_device()
        if not self._plan_valid(key):
            if torch.cuda.is_current_stream_capturing():
                return None
            self._plan = _C.build_plan(self.base_weight, self.base_scales, self.ortho_values,
                                       self.ortho_col_indices, self.ortho_row_ptr, self.in_features)
            self._plan_key = key
            self._plan_streams = set()
            if self._plan is not None:
                self._plan_event = torch.cuda.Event()
                self._plan_event.record(torch.cuda.current_stream(dev))
                self._plan_streams.add(_C._raw_stream(dev))
        if self._plan is not None:
            cur = _C._raw_stream(dev)
            if cur not in self._plan_streams and not torch.cuda.is_current_stream_capturing():
                st = torch.cuda.current_stream(dev)
                st.wait_event(self._plan_event)
                self._plan.record_stream(st)
                self._plan_streams.add(cur)
            if cur in self._plan_streams:
                v, c, r = key[0]
                self._plan_fast = (v, c, r, (v._version, v.data_ptr(), c._version, r._version), cur)
        return self._plan

    def _layer_desc(self, device):
        """The weights' C descriptor, cached until a buffer or alpha changes
        (validated when built)."""
        ts = (self.base_weight, self.base_scales, self.ortho_values, self.ortho_col_indices, self.ortho_row_ptr)
        key = (tuple((t.data_ptr(), t._version, tuple(t.shape), t.dtype) for t in ts), float(self.alpha), device)
        if getattr(self, "_desc_key", None) != key:
            self._desc = _C.make_layer(self.base_weight, self.base_scales, self.ortho_values,
                                       self.ortho_col_indices, self.ortho_row_ptr, self.in_features,
                                       self.out_features, float(self.alpha), device)
            self._desc_key = key
        return self._desc

    def _apply(self, fn, *args, **kwargs):
        self._plan = None
        self._plan_key = None
        self._plan_fast = None
        self._desc_key = None
        return super()._apply(fn, *args, **kwargs)

    def __getstate__(self):
        """Copies and pickles carry the parameters and buffers, not the
        derived caches (the C descriptor holds raw pointers, and the plan
        and its build event belong to this module's buffers); the next
        forward rebuilds them."""
        state = dict(super().__getstate__())
        for k in ("_desc", "_desc_key", "_plan_event", "_plan_streams"):
            state.pop(k, None)
        state["_plan"] = None
        state["_plan_key"] = None
        state["_plan_fast"] = None
        return state

    # --------------------------------------------------------------- forward
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        T = _lib.torch_ops()
        if T is None:
            return self._forward_ctypes(x)
        if not x.is_cuda:
            raise RuntimeError("OrthoLinear runs on a ROCm GPU only; move the module and the input "
                               "to a cuda device (the reference's CPU branch returns uninitialised memory)")
        bufs = self._buffers
        vals = bufs["ortho_values"]
        plan = None
        if self.alpha > 0 and vals.numel() > 0:
            # fast path: the same CSR tensors, unchanged, on the stream that
            # last used the plan; anything else goes through _ortho_plan
            f = self.__dict__.get("_plan_fast")
            if f is not None and f[0] is vals and f[1] is bufs["ortho_col_indices"] and \
                    f[2] is bufs["ortho_row_ptr"] and f[3] == (vals._version, vals.data_ptr(), f[1]._version,
                                                               f[2]._version) and \
                    f[4] == _C._raw_stream(vals.get_device()):
                plan = self._plan
            else:
                plan = self._ortho_plan()
        # the bias is fused into the kernel's store (same bits as `output +=
        # bias`) unless autograd must see the add
        b = self._parameters["bias"]
        fuse = b is not None and not (torch.is_grad_enabled() and b.requires_grad) and b.device == x.device
        x2 = x if x.dim() == 2 else x.reshape(-1, self.in_features)
        output = T.linear(x2, bufs["base_weight"], bufs["base_scales"], vals, bufs["ortho_col_indices"],
                          bufs["ortho_row_ptr"], self.out_features, float(self.alpha), plan,
                          b.detach() if fuse else None)
        if b is not None and not fuse:
            output += b
        return output if x.dim() == 2 else output.view(*x.shape[:-1], self.out_features)

    def _forward_ctypes(self, x: torch.Tensor) -> torch.Tensor:
        """forward through the ctypes binding (when the compiled one is absent)."""
        original_shape = x.shape
        x_flat = x.reshape(-1, self.in_features)
        batch_size = x_flat.shape[0]
        output = torch.empty(batch_size, self.out_features, device=x.device, dtype=x.dtype)
        if not x.is_cuda:
            raise RuntimeError("OrthoLinear runs on a ROCm GPU only; move the module and the input "
                               "to a cuda device (the reference's CPU branch returns uninitialised memory)")
        plan = None
        if self.alpha > 0:
            plan = self._ortho_plan()
        fuse = self.bias is not None and not (torch.is_grad_enabled() and self.bias.requires_grad) and \
            self.bias.device == x.device
        _C.forward_layer(self._layer_desc(x.device), x_flat.contiguous(), output, plan,
                         self.bias.detach().contiguous() if fuse else None)
        if self.bias is not None and not fuse:
            output += self.bias
        return output.view(*original_shape[:-1], self.out_features)

    @staticmethod
    def forward_group(modules, x: torch.Tensor):
        """``[m(x) for m in modules]`` for up to four OrthoLinear layers that
        read the same input (a block's q/k/v or gate/up projections), with
        the same results as the separate calls.  At decode batch sizes,
        layers of the same in_features and weight layout share one kernel
        launch; otherwise each runs its own.  No counterpart in the reference,
        which calls each projection's forward in turn."""
        modules = list(modules)
        if not 1 <= len(modules) <= _lib.GROUP_MAX:
            raise ValueError(f"forward_group takes 1..{_lib.GROUP_MAX} layers, got {len(modules)}")
        if not x.is_cuda:
            raise RuntimeError("OrthoLinear runs on a ROCm GPU only; move the modules and the input "
                               "to a cuda device")
        K = modules[0].in_features
        if any(m.in_features != K for m in modules):
            raise ValueError("the layers of a group must share in_features")
        x_flat = x.reshape(-1, K).contiguous()
        outs, plans, biases, late = [], [], [], []
        for m in modules:
            outs.append(torch.empty(x_flat.shape[0], m.out_features, device=x.device, dtype=x.dtype))
            plans.append(m._ortho_plan() if m.alpha > 0 else None)
            fuse = m.bias is not None and not (torch.is_grad_enabled() and m.bias.requires_grad) and \
                m.bias.device == x.device
            biases.append(m.bias.detach().contiguous() if fuse else None)
            late.append(m.bias is not None and not fuse)
        _C.forward_group([m._layer_desc(x.device) for m in modules], x_flat, outs, plans, biases)
        res = []
        for m, out, add in zip(modules, outs, late):
            if add:
                out += m.bias
            res.append(out.view(*x.shape[:-1], m.out_features))
        return res

    # ------------------------------------------------------------ checkpoints
    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        """Loads packed checkpoints of any nnz and either scale layout.

        The reference's buffers start empty and are replaced when weights are
        packed (/root/reference/torch_bind/ortho_linear.py:59-65,123-128), so
        its saved CSR has a length a fresh module cannot know: the three CSR
        buffers take the checkpoint's lengths (validated: row_ptr has
        out_features + 1 entries, 0 first, nnz last).  ``base_scales`` may be
        [out] (the reference layout: per-row scales) or [out, in/G]; the
        module takes the checkpoint's layout and sets ``group_size`` to
        match.  ``base_weight`` must be [out, in/2]."""
        N, K = self.out_features, self.in_features
        dev = self.base_weight.device

        def get(name):
            return state_dict.get(prefix + name)

        # every check first: the module is changed only once the whole
        # checkpoint has been found consistent
        bw = get("base_weight")
        if bw is not None and tuple(bw.shape) != (N, K // 2):
            error_msgs.append(f"{prefix}base_weight: expected [{N}, {K // 2}] packed INT4, got {list(bw.shape)}")
            return
        bs = get("base_scales")
        group = self.group_size
        if bs is not None:
            if bs.dim() == 1 and bs.shape[0] == N:
                group = None
            elif bs.dim() == 2 and bs.shape[0] == N and bs.shape[1] > 0 and K % bs.shape[1] == 0:
                group = K // int(bs.shape[1])
            else:
                error_msgs.append(f"{prefix}base_scales: expected [{N}] or [{N}, in/G], got {list(bs.shape)}")
                return
        vals, col, rp = get("ortho_values"), get("ortho_col_indices"), get("ortho_row_ptr")
        has_csr = vals is not None or col is not None or rp is not None
        if has_csr:
            if vals is None or col is None or rp is None:
                error_msgs.append(f"{prefix}ortho_*: the three CSR buffers must be saved together")
                return
            nnz = int(vals.numel())
            ok = col.numel() == nnz and (rp.numel() == N + 1 or (nnz == 0 and rp.numel() in (0, N + 1)))
            if ok and rp.numel() == N + 1:
                ok = int(rp[0]) == 0 and int(rp[-1]) == nnz
            if not ok:
                error_msgs.append(f"{prefix}ortho CSR: row_ptr must have {N + 1} entries from 0 to nnz and "
                                  f"col_indices nnz entries (got {rp.numel()}, {col.numel()}, nnz {nnz})")
                return
        if bs is not None:
            self.group_size = group
            self.base_scales = torch.zeros(tuple(bs.shape), dtype=torch.float16, device=dev)
        if has_csr:
            self.ortho_values = torch.zeros(nnz, dtype=torch.float16, device=dev)
            self.ortho_col_indices = torch.zeros(nnz, dtype=torch.int32, device=dev)
            self.ortho_row_ptr = torch.zeros(rp.numel(), dtype=torch.int32, device=dev)
        self._plan = None
        self._plan_key = None
        self._plan_fast = None
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    @torch.no_grad()
    def expand_scales(self, group_size: int = 128) -> "OrthoLinear":
        """Per-row scales (the reference layout) to ``group_size`` groups:
        each row's scale repeated over its groups, so every dequantised weight
        float(q) * float(s) is unchanged."""
        K = self.in_features
        if self.group_size is not None:
            raise ValueError("base_scales are already per group")
        if group_size <= 0 or K % group_size != 0:
            raise ValueError(f"group_size {group_size} must divide in_features {K}")
        self.base_scales = self.base_scales.reshape(-1, 1).repeat(1, K // group_size).contiguous()
        self.group_size = group_size
        return self

    def extra_repr(self) -> str:
        g = "row" if self.group_size is None else self.group_size
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"q_bits={self.q_bits}, group={g}, nnz={self.ortho_values.numel()}, alpha={self.alpha}")
