"""``libortho._C_ops`` for MI355X: the operator boundary of the dual GEMM.

Drop-in for the reference's torch extension, whose only entry point is

    forward(q_weight, q_scales, ortho_values, ortho_col_indices,
            ortho_row_ptr, input, output, alpha) -> None

(/root/reference/torch_bind/bindings.cpp:9-48).  Same eight positional
arguments, same meaning, ``output`` written in place, returns ``None``.
Unlike the reference binding (which cannot dispatch, bindings.cpp:39-43, and
reads FP16 buffers as FP32, :24,30) this one checks every tensor the way the
reference's draft binding intended (docs/202511271753/libortho_ops.cpp:17-20,
49-53) and raises ``RuntimeError`` with the reason, then calls the C ABI of
include/orth_hip.h on torch's current stream for ``input.device``.

Tensor contract:
  q_weight          uint8  [N, K/2]   packed signed INT4 (low nibble = even k)
  q_scales          fp16|fp32 [N] (per row) or [N, K/G] (group G)
  ortho_values      fp16|fp32 [nnz]
  ortho_col_indices int32  [nnz]
  ortho_row_ptr     int32  [N+1]  (may be empty when nnz == 0)
  input             fp16|bf16|fp32 [M, K] contiguous
  output            same dtype as input, [M, N] contiguous
  alpha             float; ortho applied iff alpha > 0 and nnz > 0

Torch appears only here, as plumbing (device pointers, dtypes, streams); the
library signatures carry plain pointers and sizes.
"""
from __future__ import annotations

import collections
import ctypes
import os
import weakref

import torch

from . import _lib

_DT = {torch.float16: _lib.DT_F16, torch.bfloat16: _lib.DT_BF16, torch.float32: _lib.DT_F32}

# the operator boundary as the reference names it, plus this build's extensions;
# forward_layer and make_layer (descriptor reuse for OrthoLinear) stay internal;
# forward_group takes make_layer descriptors (OrthoLinear.forward_group wraps it)
__all__ = ["forward", "forward_planned", "forward_group", "build_plan", "dequant", "pack_base", "pack_csr", "sieve_quantize",
           "sieve_split", "sieve_hdiag", "last_kernel", "set_kernel_policy", "get_kernel_policy", "device_info",
           "plan_cache_clear", "plan_cache_limit", "plan_cache_info"]


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _ptr(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr()) if t.numel() > 0 else None


def make_layer(q_weight: torch.Tensor, q_scales: torch.Tensor, ortho_values: torch.Tensor,
               ortho_col_indices: torch.Tensor, ortho_row_ptr: torch.Tensor, K: int, N: int,
               alpha: float, device: torch.device) -> _lib.OrthHipLayer:
    """Validate the weight tensors and describe them as an orth_hip_layer_t."""
    for name, t in (("q_weight", q_weight), ("q_scales", q_scales),
                    ("ortho_values", ortho_values), ("ortho_col_indices", ortho_col_indices),
                    ("ortho_row_ptr", ortho_row_ptr)):
        _req(isinstance(t, torch.Tensor), f"{name} must be a tensor")
        _req(t.numel() == 0 or t.device == device,
             f"{name} is on {t.device} but input is on {device}")
        _req(t.is_contiguous(), f"{name} must be contiguous")
    _req(K > 0 and K % 2 == 0, f"in_features must be positive and even (got {K})")
    _req(q_weight.dtype == torch.uint8, f"q_weight must be uint8 (got {q_weight.dtype})")
    _req(tuple(q_weight.shape) == (N, K // 2),
         f"q_weight must have shape ({N}, {K // 2}) (got {tuple(q_weight.shape)})")
    _req(q_scales.dtype in (torch.float16, torch.float32),
         f"q_scales must be float16 or float32 (got {q_scales.dtype})")
    if q_scales.dim() == 1:
        _req(q_scales.shape[0] == N, f"q_scales must have {N} rows (got {tuple(q_scales.shape)})")
        groups = 1
    else:
        _req(q_scales.dim() == 2 and q_scales.shape[0] == N,
             f"q_scales must be [{N}] or [{N}, K/G] (got {tuple(q_scales.shape)})")
        groups = int(q_scales.shape[1])
        _req(groups >= 1 and K % groups == 0,
             f"q_scales has {groups} groups, which does not divide in_features {K}")
    nnz = int(ortho_values.numel())
    _req(ortho_col_indices.numel() == nnz,
         f"ortho_col_indices has {ortho_col_indices.numel()} entries, ortho_values {nnz}")
    if nnz > 0:
        _req(ortho_values.dtype in (torch.float16, torch.float32),
             f"ortho_values must be float16 or float32 (got {ortho_values.dtype})")
        _req(ortho_col_indices.dtype == torch.int32,
             f"ortho_col_indices must be int32 (got {ortho_col_indices.dtype})")
        _req(ortho_row_ptr.dtype == torch.int32,
             f"ortho_row_ptr must be int32 (got {ortho_row_ptr.dtype})")
        _req(ortho_row_ptr.numel() == N + 1,
             f"ortho_row_ptr must have {N + 1} entries (got {ortho_row_ptr.numel()})")
    layer = _lib.OrthHipLayer()
    layer.base.q_weight = _ptr(q_weight)
    layer.base.q_scales = _ptr(q_scales)
    layer.base.q_bits = 4
    layer.base.scale_dtype = _DT[q_scales.dtype]
    layer.base.scale_groups = groups
    layer.base.in_features = K
    layer.base.out_features = N
    layer.ortho.count = nnz
    if nnz > 0:
        layer.ortho.row_ptr = _ptr(ortho_row_ptr)
        layer.ortho.col_indices = _ptr(ortho_col_indices)
        layer.ortho.values = _ptr(ortho_values)
        layer.ortho.value_dtype = _DT[ortho_values.dtype]
    layer.alpha = float(alpha)
    return layer


def _check_io(input: torch.Tensor, output: torch.Tensor):
    _req(isinstance(input, torch.Tensor) and isinstance(output, torch.Tensor),
         "input and output must be tensors")
    _req(input.is_cuda, "input must be on a ROCm GPU (libortho_amd has no CPU path)")
    _req(output.device == input.device, "output must be on the same device as input")
    _req(input.dim() == 2 and output.dim() == 2, "input and output must be 2-D [M, K] / [M, N]")
    _req(input.dtype in _DT, f"input dtype {input.dtype} is not float16, bfloat16 or float32")
    _req(output.dtype == input.dtype,
         f"output dtype {output.dtype} must equal input dtype {input.dtype}")
    _req(input.is_contiguous() and output.is_contiguous(), "input and output must be contiguous")
    _req(output.shape[0] == input.shape[0],
         f"output has {output.shape[0]} rows, input {input.shape[0]}")


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _raw_stream(dev_index: int) -> int:
    """The current stream of device ``dev_index`` as its raw handle (cheap:
    no Stream object)."""
    get = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    return get(dev_index) if get is not None else torch.cuda.current_stream(dev_index).cuda_stream


def forward(q_weight, q_scales, ortho_values, ortho_col_indices, ortho_row_ptr, input, output,
            alpha) -> None:
    """y = Base(x) + alpha * Ortho(x), written into ``output`` in place.

    The reference's operator carries no plan, so with alpha > 0 this entry
    keeps one per weight set (:class:`_PlanCache`): the first call on a set
    builds it, later calls take the planned kernels (at 2,048 tokens of c3
    ~100 instead of ~163 µs an eager call, which otherwise builds a
    temporary plan each time). Results are those of ``forward_planned`` with
    that plan; calls under graph capture take none.

    The first call on a weight set blocks until its plan is built (the build
    reads the plan's flags back to the host).  The cache holds up to 4,096
    plans and 8 GiB of device memory (a plan is ~12 % of its INT4 weights),
    least recently used out; :func:`plan_cache_limit` changes the bounds (0
    entries: no cache, every call reads the CSR), :func:`plan_cache_clear`
    frees it, :func:`plan_cache_info` reports it."""
    plan = _PLANS.lookup((q_weight, q_scales, ortho_values, ortho_col_indices, ortho_row_ptr), input,
                         alpha)
    T = _lib.torch_ops()
    if T is not None:
        T.forward_planned(q_weight, q_scales, ortho_values, ortho_col_indices, ortho_row_ptr, input, output,
                          float(alpha), plan)
        return
    forward_planned(q_weight, q_scales, ortho_values, ortho_col_indices, ortho_row_ptr, input,
                    output, alpha, plan)


def plan_cache_clear() -> None:
    """Drops every plan the 8-argument :func:`forward` keeps (their device
    memory is freed once the streams that used them are done with it)."""
    _PLANS.clear()


def plan_cache_limit(entries=None, max_bytes=None) -> tuple:
    """Sets the bounds of the 8-argument :func:`forward`'s plan cache (None
    keeps a bound) and returns them as (entries, bytes); least recently used
    plans beyond the new bounds are dropped at once.  Defaults: 4,096 plans
    and 8 GiB, or the environment's LIBORTHO_PLAN_CACHE_ENTRIES and
    LIBORTHO_PLAN_CACHE_BYTES; entries=0 turns the cache off."""
    if entries is not None:
        _req(int(entries) >= 0, "entries must be >= 0")
        _PLANS.max_entries = int(entries)
    if max_bytes is not None:
        _req(int(max_bytes) >= 0, "max_bytes must be >= 0")
        _PLANS.max_bytes = int(max_bytes)
    _PLANS.trim()
    return _PLANS.max_entries, _PLANS.max_bytes


def plan_cache_info() -> dict:
    """Entries and device bytes the 8-argument :func:`forward`'s plan cache holds, and its bounds."""
    return {"entries": len(_PLANS), "bytes": _PLANS._bytes, "max_entries": _PLANS.max_entries,
            "max_bytes": _PLANS.max_bytes}


class _PlanCache:
    """Ortho plans of the weight sets the 8-argument ``forward`` has seen.

    An entry holds weak references to its five tensors and is valid only
    while the same tensor objects are alive with unchanged versions, data
    pointers and shapes (an in-place write bumps ``_version``; a freed tensor
    drops its entries).  Bounded by MAX entries and MAX_BYTES of plans (a
    model's every layer fits: a plan is ~12 % of its INT4 weights), least
    recently used first out.  A plan
    built on one stream is used on another only after that stream has waited
    on the build, and its memory is recorded on that stream, so freeing it
    waits for the stream's work.  Under graph capture no plan is handed out
    (a graph would keep the pointer of a plan this cache may free): captured
    calls read the CSR as the reference's operator does."""

    MAX = 4096
    MAX_BYTES = 8 << 30

    def __init__(self):
        self._d = collections.OrderedDict()
        self._bytes = 0
        self.max_entries = int(os.environ.get("LIBORTHO_PLAN_CACHE_ENTRIES", self.MAX))
        self.max_bytes = int(os.environ.get("LIBORTHO_PLAN_CACHE_BYTES", self.MAX_BYTES))

    def __len__(self):
        return len(self._d)

    def clear(self):
        self._d.clear()
        self._bytes = 0

    def trim(self):
        while self._d and (len(self._d) > self.max_entries or self._bytes > self.max_bytes):
            self._drop(next(iter(self._d)))

    def _drop(self, key):
        e = self._d.pop(key, None)
        if e is not None:
            self._bytes -= e["plan"].numel()

    @staticmethod
    def _sig(ts):
        return tuple((t._version, t.data_ptr(), t.shape, t.dtype) for t in ts)

    def lookup(self, ts, input, alpha):
        """The plan for weight tensors ``ts`` (q, scales, values, columns,
        row pointers) and ``input``, or None."""
        try:
            if not (float(alpha) > 0 and ts[2].numel() > 0 and input.is_cuda and input.dim() == 2):
                return None
            dev = input.get_device()
            key = (id(ts[0]), id(ts[1]), id(ts[2]), id(ts[3]), id(ts[4]), int(input.shape[1]), dev)
        except (AttributeError, TypeError, ValueError):
            return None
        if torch.cuda.is_current_stream_capturing():
            return None  # a graph would keep the pointer of a plan this cache may free
        if self.max_entries == 0:
            return None
        e = self._d.get(key)
        if e is not None:
            r = e["refs"]
            if (r[0]() is ts[0] and r[1]() is ts[1] and r[2]() is ts[2] and r[3]() is ts[3] and r[4]() is ts[4]
                    and e["sig"] == self._sig(ts)):
                self._d.move_to_end(key)
                cur = _raw_stream(dev)
                if cur not in e["streams"]:  # first use on this stream: order it after the build,
                    st = torch.cuda.current_stream(dev)  # and keep the plan's memory from reuse
                    st.wait_event(e["event"])              # until this stream's work on it is done
                    e["plan"].record_stream(st)
                    e["streams"].add(cur)
                return e["plan"]
            self._drop(key)
        if not all(isinstance(t, torch.Tensor) and t.is_cuda and t.get_device() == dev for t in ts):
            return None  # forward_planned raises the reason
        try:
            plan = build_plan(*ts, key[5])
        except (RuntimeError, ValueError):
            return None
        if plan is None:
            return None
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(dev))
        owner = weakref.ref(self)

        def drop(_r, key=key, owner=owner):
            c = owner()
            if c is not None:
                c._drop(key)
        self._d[key] = {"refs": tuple(weakref.ref(t, drop) for t in ts), "sig": self._sig(ts), "plan": plan,
                        "event": ev, "streams": {_raw_stream(dev)}}
        self._bytes += plan.numel()
        while len(self._d) > 1 and (len(self._d) > self.max_entries or self._bytes > self.max_bytes):
            self._drop(next(iter(self._d)))
        return plan


_PLANS = _PlanCache()


def forward_planned(q_weight, q_scales, ortho_values, ortho_col_indices, ortho_row_ptr, input,
                    output, alpha, plan, bias=None) -> None:
    """``forward`` with an ortho plan from :func:`build_plan` (or None) and,
    optionally, the bias [N] fused into the store (the bits of ``output +=
    bias`` after the kernel)."""
    T = _lib.torch_ops()
    if T is not None:
        T.forward_planned(q_weight, q_scales, ortho_values, ortho_col_indices, ortho_row_ptr, input, output,
                          float(alpha), plan, bias)
        return
    _check_io(input, output)
    K, N = int(input.shape[1]), int(output.shape[1])
    dev = input.device
    layer = make_layer(q_weight, q_scales, ortho_values, ortho_col_indices, ortho_row_ptr, K, N,
                       float(alpha), dev)
    L = _lib.lib()
    has_plan = plan is not None and plan.numel() > 0
    if has_plan:
        _req(plan.device == dev and plan.dtype == torch.uint8, "plan must be a uint8 tensor on input's device")
    with torch.cuda.device(dev):
        if bias is not None:
            _req(bias.device == dev and bias.dtype in _DT and bias.numel() == N and bias.is_contiguous(),
                 f"bias must be a contiguous float tensor of {N} elements on input's device")
            rc = L.orth_layer_forward_hip_ex(ctypes.byref(layer), _ptr(plan) if has_plan else None,
                                             plan.numel() if has_plan else 0, _ptr(bias), _DT[bias.dtype],
                                             _ptr(input), _ptr(output), int(input.shape[0]),
                                             _DT[input.dtype], _stream(dev))
        elif has_plan:
            rc = L.orth_layer_forward_hip_planned(ctypes.byref(layer), _ptr(plan), plan.numel(),
                                                  _ptr(input), _ptr(output), int(input.shape[0]),
                                                  _DT[input.dtype], _stream(dev))
        else:
            rc = L.orth_layer_forward_hip(ctypes.byref(layer), _ptr(input), _ptr(output),
                                          int(input.shape[0]), _DT[input.dtype], _stream(dev))
    _lib.check(rc)


def forward_layer(layer, input, output, plan=None, bias=None) -> None:
    """``forward_planned`` with a descriptor from :func:`make_layer` built
    earlier for the same, unchanged weight tensors (the caller keeps them
    alive): skips re-validating and re-describing the weights on every call."""
    _check_io(input, output)
    _req(int(input.shape[1]) == layer.base.in_features,
         f"input has {input.shape[1]} columns, the layer {layer.base.in_features} in_features")
    _req(int(output.shape[1]) == layer.base.out_features,
         f"output has {output.shape[1]} columns, the layer {layer.base.out_features} out_features")
    dev = input.device
    L = _lib.lib()
    has_plan = plan is not None and plan.numel() > 0
    if has_plan:
        _req(plan.device == dev and plan.dtype == torch.uint8, "plan must be a uint8 tensor on input's device")
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if bias is not None:
        _req(bias.device == dev and bias.dtype in _DT and bias.numel() == output.shape[1] and bias.is_contiguous(),
             "bias must be a contiguous float tensor of out_features elements on input's device")

    def call():
        return L.orth_layer_forward_hip_ex(ctypes.byref(layer), _ptr(plan) if has_plan else None,
                                           plan.numel() if has_plan else 0,
                                           _ptr(bias) if bias is not None else None,
                                           _DT[bias.dtype] if bias is not None else 0, _ptr(input),
                                           _ptr(output), int(input.shape[0]), _DT[input.dtype], stream)
    if dev.index == torch.cuda.current_device():
        rc = call()
    else:
        with torch.cuda.device(dev):
            rc = call()
    _lib.check(rc)


def forward_group(layers, input, outputs, plans=None, biases=None) -> None:
    """Several layers over one input, ``outputs[l] = layers[l](input)``, in a
    single decode launch when the layers allow it (same in_features, scale
    layout, ortho mode; decode-sized batches), else one launch per layer.
    ``layers``: descriptors from :func:`make_layer`, as for
    :func:`forward_layer`; ``plans`` / ``biases``: lists of the same length
    with None entries for none."""
    n = len(layers)
    _req(1 <= n <= _lib.GROUP_MAX, f"a group holds 1..{_lib.GROUP_MAX} layers, got {n}")
    _req(len(outputs) == n, f"{len(outputs)} outputs for {n} layers")
    plans = list(plans) if plans is not None else [None] * n
    biases = list(biases) if biases is not None else [None] * n
    _req(len(plans) == n and len(biases) == n, "plans and biases must have one entry per layer")
    dev = input.device
    for layer, out, plan, bias in zip(layers, outputs, plans, biases):
        _check_io(input, out)
        _req(int(input.shape[1]) == layer.base.in_features,
             f"input has {input.shape[1]} columns, a layer {layer.base.in_features} in_features")
        _req(int(out.shape[1]) == layer.base.out_features,
             f"an output has {out.shape[1]} columns, its layer {layer.base.out_features} out_features")
        if plan is not None and plan.numel() > 0:
            _req(plan.device == dev and plan.dtype == torch.uint8, "plan must be a uint8 tensor on input's device")
        if bias is not None:
            _req(bias.device == dev and bias.dtype in _DT and bias.numel() == out.shape[1] and bias.is_contiguous(),
                 "bias must be a contiguous float tensor of out_features elements on input's device")
    has = [p is not None and p.numel() > 0 for p in plans]
    c_layers = (ctypes.c_void_p * n)(*[ctypes.addressof(layer) for layer in layers])
    c_plans = (ctypes.c_void_p * n)(*[p.data_ptr() if h else None for p, h in zip(plans, has)])
    c_pbytes = (ctypes.c_int64 * n)(*[p.numel() if h else 0 for p, h in zip(plans, has)])
    c_bias = (ctypes.c_void_p * n)(*[b.data_ptr() if b is not None else None for b in biases])
    c_bdt = (ctypes.c_int32 * n)(*[_DT[b.dtype] if b is not None else 0 for b in biases])
    c_out = (ctypes.c_void_p * n)(*[o.data_ptr() if o.numel() > 0 else None for o in outputs])
    L = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def call():
        return L.orth_layers_forward_hip(c_layers, c_plans, c_pbytes, c_bias, c_bdt, n, _ptr(input), c_out,
                                         int(input.shape[0]), _DT[input.dtype], stream)
    if dev.index == torch.cuda.current_device():
        rc = call()
    else:
        with torch.cuda.device(dev):
            rc = call()
    _lib.check(rc)


def build_plan(q_weight, q_scales, ortho_values, ortho_col_indices, ortho_row_ptr,
               in_features: int):
    """Build the ortho plan (derived layout of the CSR used by the prefill
    kernel) into a new uint8 tensor on the weights' device.  Returns None when
    the layer has no ortho entries or its shape takes no plan."""
    dev = q_weight.device
    _req(dev.type == "cuda", "build_plan needs the weights on a ROCm GPU")
    N = int(q_weight.shape[0])
    layer = make_layer(q_weight, q_scales, ortho_values, ortho_col_indices, ortho_row_ptr,
                       int(in_features), N, 1.0, dev)
    L = _lib.lib()
    nbytes = L.orth_ortho_plan_bytes(ctypes.byref(layer))
    if nbytes <= 0:
        return None
    plan = torch.empty(int(nbytes), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.check(L.orth_ortho_plan_build(ctypes.byref(layer), _ptr(plan), plan.numel(),
                                           _stream(dev)))
    return plan


def dequant(q_weight, q_scales, in_features: int) -> torch.Tensor:
    """FP32 [N, K] dequantised Base, float(q) * float(s), on the GPU."""
    dev = q_weight.device
    _req(dev.type == "cuda", "dequant needs the weights on a ROCm GPU")
    N = int(q_weight.shape[0])
    empty_f = torch.empty(0, dtype=torch.float16, device=dev)
    empty_i = torch.empty(0, dtype=torch.int32, device=dev)
    layer = make_layer(q_weight, q_scales, empty_f, empty_i, empty_i, int(in_features), N, 0.0, dev)
    out = torch.empty((N, int(in_features)), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().orth_base_dequant_hip(ctypes.byref(layer), _ptr(out), _stream(dev)))
    return out


def pack_base(base_weight: torch.Tensor, group_size=None, base_scales=None):
    """INT4 quantisation and nibble packing of dense ``base_weight`` [N, K]
    on the GPU: (q uint8 [N, K/2], scales float16 [N] or [N, K/G]), the
    results of load_from_weights' torch ops on a GPU tensor
    (/root/reference/torch_bind/ortho_linear.py:89-120)."""
    dev = base_weight.device
    _req(dev.type == "cuda", "pack_base needs the weights on a ROCm GPU")
    _req(base_weight.dim() == 2 and base_weight.dtype in _DT,
         "base_weight must be a 2-D float16, bfloat16 or float32 tensor")
    w = base_weight.contiguous()
    N, K = int(w.shape[0]), int(w.shape[1])
    G = K if group_size is None else int(group_size)
    _req(K % 2 == 0 and G > 0 and G % 2 == 0 and K % G == 0,
         f"in_features ({K}) must be even and group_size ({G}) even and dividing it")
    s_in = None
    if base_scales is not None:
        _req(base_scales.dtype in _DT and base_scales.device == dev and base_scales.numel() == N * (K // G),
             "base_scales must be float16/bfloat16/float32 on the weights' device with N * K/G elements")
        s_in = base_scales.contiguous()
    q = torch.empty((N, K // 2), dtype=torch.uint8, device=dev)
    # [N] for per-row scales (group_size None, the reference layout), else [N, K/G]
    scales = torch.empty((N,) if group_size is None else (N, K // G), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().orth_pack_base_hip(
            _ptr(w), _DT[w.dtype], N, K, G, _ptr(s_in) if s_in is not None else None,
            _DT[s_in.dtype] if s_in is not None else 0, _ptr(q), _ptr(scales), _stream(dev)))
    return q, scales


def pack_base_path(base_weight: torch.Tensor, group_size, q: torch.Tensor) -> int:
    """Kernel pack_base takes: 1 per-group waves, 2 per-row workgroups, 3 fallback."""
    K = int(base_weight.shape[1])
    return _lib.lib().orth_pack_base_path(_ptr(base_weight), _DT[base_weight.dtype], K,
                                          K if group_size is None else int(group_size), _ptr(q))


def pack_csr(ortho_weight: torch.Tensor, values_dtype=None, use_mask: bool = True):
    """CSR of the nonzeros of dense ``ortho_weight`` [N, K] built on the GPU:
    (row_ptr int32 [N+1], col int32 [nnz], values [nnz] in ``values_dtype``,
    default the weight's dtype), as pack_ortho_sparse(W, "csr")
    (/root/reference/tools/sieve.py:119-152).  Reads nnz back to the host.
    With ``use_mask`` the first pass records the nonzero pattern in a
    temporary mask and the second reads only the nonzero elements."""
    dev = ortho_weight.device
    _req(dev.type == "cuda", "pack_csr needs the weights on a ROCm GPU")
    _req(ortho_weight.dim() == 2 and ortho_weight.dtype in _DT,
         "ortho_weight must be a 2-D float16, bfloat16 or float32 tensor")
    w = ortho_weight.contiguous()
    N, K = int(w.shape[0]), int(w.shape[1])
    vdt = w.dtype if values_dtype is None else values_dtype
    _req(vdt in _DT, f"values dtype {vdt} is not float16, bfloat16 or float32")
    row_ptr = torch.empty(N + 1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        L = _lib.lib()
        mb = int(L.orth_pack_csr_mask_bytes(_ptr(w), _DT[w.dtype], N, K)) if use_mask else 0
        _req(mb >= 0, _lib.last_error())
        mask = torch.empty(mb, dtype=torch.uint8, device=dev) if mb > 0 else None
        mp = _ptr(mask) if mask is not None else None
        _lib.check(L.orth_pack_csr_rows_hip(_ptr(w), _DT[w.dtype], N, K, _ptr(row_ptr), mp, mb, _stream(dev)))
        nnz = int(row_ptr[N].item())  # synchronises the stream
        _req(nnz >= 0, "more than 2^31 - 1 nonzeros")
        col = torch.empty(nnz, dtype=torch.int32, device=dev)
        vals = torch.empty(nnz, dtype=vdt, device=dev)
        if nnz > 0:
            _lib.check(L.orth_pack_csr_fill_hip(_ptr(w), _DT[w.dtype], N, K, _ptr(row_ptr), mp, mb, _ptr(col),
                                                _ptr(vals), _DT[vdt], _stream(dev)))
    return row_ptr, col, vals


SIEVE_IEEE_DIV = 1  # ORTH_SIEVE_IEEE_DIV: divide by host scalars as torch does on a CPU tensor


def _sieve_flags(ieee_div: bool) -> int:
    return SIEVE_IEEE_DIV if ieee_div else 0


def sieve_quantize(weight: torch.Tensor, ieee_div: bool = False) -> torch.Tensor:
    """quantize_int4 (/root/reference/tools/sieve.py:13-23) of a 2-D GPU
    tensor with the library's kernel: same dtype and shape as ``weight``.
    ``ieee_div`` divides by the host scalar 7 as torch does on a CPU tensor
    (IEEE division) rather than as on a GPU tensor (a product with the FP32
    reciprocal)."""
    _req(weight.is_cuda and weight.dim() == 2 and weight.dtype in _DT,
         "sieve_quantize needs a 2-D float16, bfloat16 or float32 tensor on a ROCm GPU")
    w = weight.contiguous()
    out = torch.empty_like(w)
    if w.numel() == 0:
        return out
    with torch.cuda.device(w.device):
        _lib.check(_lib.lib().orth_sieve_quantize_hip(_ptr(w), _DT[w.dtype], int(w.shape[0]), int(w.shape[1]),
                                                      _ptr(out), _sieve_flags(ieee_div), _stream(w.device)))
    return out


def sieve_split(weight: torch.Tensor, H_inv: torch.Tensor, curvature_thresh: float = 10.0,
                sparsity_target=None, ieee_div: bool = False):
    """hessian_sieve (/root/reference/tools/sieve.py:25-76) with the
    library's kernels: (w_base, w_ortho), both of ``weight``'s dtype
    (``ieee_div`` as in :func:`sieve_quantize`)."""
    _req(weight.is_cuda and weight.dim() == 2 and weight.dtype in _DT,
         "sieve_split needs a 2-D float16, bfloat16 or float32 weight on a ROCm GPU")
    _req(H_inv.device == weight.device and H_inv.dtype in _DT and H_inv.dim() in (1, 2),
         "H_inv must be a 1-D or 2-D float tensor on the weight's device")
    w = weight.contiguous()
    N, K = int(w.shape[0]), int(w.shape[1])
    h = torch.diagonal(H_inv) if H_inv.dim() > 1 else H_inv
    if h.numel() == 1:
        h_stride = 0
    else:
        _req(h.numel() == K, f"H_inv has {h.numel()} diagonal entries, the weight {K} columns")
        h_stride = int(h.stride(0))
    score_dt = torch.promote_types(w.dtype, h.dtype)
    w_base = torch.empty_like(w)
    w_ortho = torch.empty_like(w)
    if w.numel() == 0:
        return w_base, w_ortho
    score = torch.empty(N * K, dtype=torch.float32, device=w.device)
    L = _lib.lib()
    use_rank = sparsity_target is not None
    rank = int(sparsity_target * (N * K)) if use_rank else 0
    sel = torch.empty(int(L.orth_sieve_select_bytes()), dtype=torch.uint8, device=w.device)
    with torch.cuda.device(w.device):
        _lib.check(L.orth_sieve_split_hip(_ptr(w), _DT[w.dtype], N, K, ctypes.c_void_p(h.data_ptr()), _DT[h.dtype],
                                          h_stride, _DT[score_dt], 1 if use_rank else 0, rank,
                                          float(curvature_thresh) if not use_rank else 0.0, _ptr(w_base),
                                          _ptr(w_ortho), _ptr(score), _ptr(sel), _sieve_flags(ieee_div),
                                          _stream(w.device)))
    return w_base, w_ortho


def sieve_hdiag(inputs: torch.Tensor, ieee_div: bool = False) -> torch.Tensor:
    """compute_hessian_diag_approx (/root/reference/tools/sieve.py:79-95),
    diag(X^T X) / n + 1e-6, of a 2-D GPU tensor with the library's kernels
    (``ieee_div``: the division by n as on a CPU tensor)."""
    _req(inputs.is_cuda and inputs.dim() == 2 and inputs.dtype in _DT,
         "sieve_hdiag needs a 2-D float16, bfloat16 or float32 tensor on a ROCm GPU")
    x = inputs.contiguous()
    n, K = int(x.shape[0]), int(x.shape[1])
    _req(n > 0 and K > 0, "inputs must have rows and columns")
    L = _lib.lib()
    ws_n = int(L.orth_sieve_hdiag_workspace(n, K))
    ws = torch.empty(ws_n, dtype=torch.float32, device=x.device)
    out = torch.empty(K, dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(L.orth_sieve_hdiag_hip(_ptr(x), _DT[x.dtype], n, K, _ptr(ws), ws_n, _ptr(out),
                                          _sieve_flags(ieee_div), _stream(x.device)))
    return out


def last_kernel() -> str:
    """Kernel used by this thread's last forward: decode, skinny (5..64
    tokens), prefill, general, or decode_group (one decode launch for the
    layers of a :func:`forward_group` call)."""
    return _lib.last_kernel()


set_kernel_policy = _lib.set_kernel_policy
get_kernel_policy = _lib.get_kernel_policy
device_info = _lib.device_info
