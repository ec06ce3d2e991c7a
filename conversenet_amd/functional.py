"""Tensor-level wrappers over the HIP C ABI (fp32, HIP device tensors only, forward only).

Each wrapper validates shapes the way the reference does (TORCH_CHECK -> RuntimeError,
Converse2D/torch_converse2d/converse2d.cpp:167-172), makes inputs contiguous like the reference op
(:174-177), allocates outputs and workspace through torch's caching allocator and enqueues the
kernels on torch's current stream.  No CPU fallback exists here: a missing library raises.
"""
from __future__ import annotations

import os
import threading

import torch

from . import _lib, composite

# The op is callable from any host thread (the reference guards its OTF cache with a mutex,
# converse2d.cpp:56,70,90): the workspace map, the plan memo and the table cache each take a lock
# around their dict updates.  Kernel launches and table builds run outside the locks.
_ws_cache: dict = {}
_ws_lock = threading.Lock()


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _need_hip(*ts):
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("conversenet_amd HIP path needs tensors on a HIP device")
        if t.dtype != torch.float32:
            raise RuntimeError("conversenet_amd HIP path computes in float32")


def _workspace(dev, nbytes: int, stream=None):
    """A reusable uint8 scratch tensor per (device, stream); grows monotonically.  stream: the current
    stream's handle when the caller has it already."""
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream if stream is None else stream)
    with _ws_lock:
        buf = _ws_cache.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
            _ws_cache[key] = buf
    return buf


def release_workspace():
    with _ws_lock:
        _ws_cache.clear()


class TableCache:
    """LRU cache of transfer tables, the counterpart of the reference's OTF cache (converse2d.cpp:52-102).

    Key: the psf and bias tensors (data pointer and version counter), eps, the geometry, the route
    (which fixes the table's layout) and the device.  Entries hold strong references to psf and bias,
    so a cached address cannot be reused by another tensor while the entry lives.  An in-place update
    (optimizer step, load_state_dict) bumps the version and misses; the entry of the older version is
    dropped then, so updates leave no dead tables behind.  Writes through `.data` (p.data.copy_(...),
    p.data.mul_(...)) do not bump the version counter: call torch.ops.converse2d.clear_cache() after such
    a write, as with the reference's cache, which keys on the data pointer alone.

    Callers cache only tables that can be hit again (see `cacheable`).  Bounded by the reference's
    64 entries and by bytes."""

    def __init__(self, max_entries=64, max_bytes=4 << 30):
        from collections import OrderedDict

        self.entries = OrderedDict()
        self._lock = threading.RLock()
        self.latest = {}  # key without version counters -> full key
        self.max_entries = max_entries
        self.max_bytes = max_bytes
        self.bytes = 0
        self.hits = 0
        self.misses = 0

    @staticmethod
    def _stem(key):
        return key[:2] + key[3:4] + key[5:]

    def get(self, key):
        with self._lock:
            e = self.entries.get(key)
            if e is None:
                self.misses += 1
                return None
            self.entries.move_to_end(key)
            self.hits += 1
            return e[0]

    def _drop(self, key):  # caller holds self._lock
        t, _ = self.entries.pop(key)
        self.bytes -= t.numel()
        stem = self._stem(key)
        if self.latest.get(stem) == key:
            del self.latest[stem]

    def put(self, key, table, refs):
        with self._lock:
            old = self.latest.get(self._stem(key))
            if old is not None and old in self.entries:
                self._drop(old)  # the same tensors at an older version: never hit again
            prev = self.entries.pop(key, None)
            if prev is not None:  # another thread built the same table meanwhile: keep one copy
                self.bytes -= prev[0].numel()
            self.entries[key] = (table, refs)
            self.latest[self._stem(key)] = key
            self.bytes += table.numel()
            while self.entries and (len(self.entries) > self.max_entries or self.bytes > self.max_bytes):
                self._drop(next(iter(self.entries)))

    def clear(self):
        with self._lock:
            self.entries.clear()
            self.latest.clear()
            self.bytes = 0


table_cache = TableCache()


def cacheable(weight, bias) -> bool:
    """Whether a table for (weight, bias) can be hit by a later call: not for inference tensors (no
    version counter; in inference mode they are fresh activations), and not while autograd tracks the
    parameters (an optimizer step changes them before the next call; the reference bypasses its cache
    then, converse2d.cpp:60,68,88)."""
    for t in (weight, bias):
        if t.is_inference() or (torch.is_grad_enabled() and t.requires_grad):
            return False
    return True


def _cache_key(kind, weight, bias, eps, geo, route, dev):
    return (kind, weight.data_ptr(), weight._version, bias.data_ptr(), bias._version, float(eps), geo, route,
            dev.index)


_plan_memo: dict = {}
_plan_lock = threading.Lock()


def _module_plan(lib, B, C, H, W, pb, kh, kw, s, p):
    """(route, table bytes, scratch bytes) of a module-level call: the library's answers depend only on
    the geometry and CVN_DISABLE_FUSED, so they are asked once per geometry (three queries cost about as
    much host time as a small layer's kernels)."""
    key = (B, C, H, W, pb, kh, kw, s, p, os.environ.get("CVN_DISABLE_FUSED"))
    plan = _plan_memo.get(key)
    if plan is None:
        route = lib.cvn_converse2d_route(B, C, H, W, pb, kh, kw, s, p)
        if route < 0:
            _lib.check(route, "converse2d_fused")
        plan = (route, lib.cvn_converse2d_table_bytes(B, C, H, W, pb, kh, kw, s, p, route),
                lib.cvn_converse2d_scratch_bytes(B, C, H, W, pb, kh, kw, s, p, route))
        with _plan_lock:
            if len(_plan_memo) >= 1024:
                _plan_memo.clear()
            _plan_memo[key] = plan
    return plan


def module_route(shape, weight, scale, padding):
    """The library's route (_lib.ROUTE_*) for a module-level call on an input of `shape` (B, C, H, W)."""
    B, C, H, W = (int(v) for v in shape)
    return _module_plan(_lib.load(), B, C, H, W, int(weight.shape[0]), int(weight.shape[2]), int(weight.shape[3]),
                        int(scale), int(padding))[0]


def converse2d_fused(x, weight, bias, scale=1, padding=2, padding_mode="circular", eps=1e-5, act=None,
                     cache=True):
    """Converse2D.forward (util_converse.py:142-192) in one library call: pad, solve, crop.

    x (B,C,H,W); weight (1,C,kh,kw) or (B,C,kh,kw) (per-sample psf, as ConvReverseDataNet);
    bias (1,C,1,1) or (C,).  act='gelu' applies exact GELU to the output on store.  cache=True keeps
    the transfer table of a shared psf (psf batch 1) for reuse while weight and bias are unchanged
    (version-checked); per-sample psfs are activations that change every call and are not cached."""
    lib = _lib.load()
    _need_hip(x, weight, bias)
    if x.dim() != 4:
        raise RuntimeError("x must be (B,C,H,W)")
    B, C, H, W = x.shape
    if weight.dim() != 4 or weight.shape[1] != C or weight.shape[0] not in (1, B):
        raise RuntimeError("weight must be (1,C,kh,kw) or (B,C,kh,kw)")
    if bias.numel() != C:
        raise RuntimeError("bias must hold C values")
    if padding_mode not in _lib.PAD_MODES:
        raise ValueError(f"unknown padding_mode {padding_mode!r}")
    s = int(scale)
    if s < 1:
        raise RuntimeError("scale must be >= 1")
    kh, kw = int(weight.shape[2]), int(weight.shape[3])
    pb = int(weight.shape[0])
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    dev = x.device
    out = torch.empty((B, C, H * s, W * s), dtype=torch.float32, device=dev)
    if B == 0:
        return out
    p = int(padding)
    route, tb, sb = _module_plan(lib, B, C, H, W, pb, kh, kw, s, p)
    st = _stream(dev)
    key = None
    table = None
    if cache and pb == 1 and cacheable(weight, bias):
        key = _cache_key("module", weight, bias, eps, (C, H, W, kh, kw, s, p), route, dev)
        table = table_cache.get(key)
    if table is None:
        wc = weight.contiguous()
        bc = bias.contiguous()
        table = torch.empty(tb, dtype=torch.uint8, device=dev)
        _lib.check(lib.cvn_converse2d_table_f32(wc.data_ptr(), pb, kh, kw, bc.data_ptr(), float(eps), B, C, H, W,
                                                s, p, route, table.data_ptr(), tb, st), "converse2d transfer table")
        if key is not None:
            table_cache.put(key, table, (weight, bias))
    scratch = _workspace(dev, sb, st) if sb > 0 else None
    rc = lib.cvn_converse2d_apply_f32(
        x.data_ptr(), B, C, H, W, pb, kh, kw, s, p, _lib.PAD_MODES[padding_mode],
        _lib.ACT_GELU if act == "gelu" else _lib.ACT_NONE, route, table.data_ptr(), tb,
        scratch.data_ptr() if scratch is not None else None, sb, out.data_ptr(), st)
    _lib.check(rc, "converse2d_fused")
    return out


def supported(x, weight, scale, padding, grad_x=False, grad_weight=False, shape=None) -> bool:
    """Whether the library's forward (and the requested backward) serves this geometry
    (cvn_converse2d_supported); shapes it does not serve go to the PyTorch composition.  shape
    (B, C, H, W) stands in for x's shape when given."""
    lib = _lib.load()
    if weight.dim() != 4 or (shape is None and x.dim() != 4):
        return False
    B, C, H, W = shape if shape is not None else x.shape
    return lib.cvn_converse2d_supported(B, C, H, W, int(weight.shape[0]), int(weight.shape[2]),
                                        int(weight.shape[3]), int(scale), int(padding), int(bool(grad_x)),
                                        int(bool(grad_weight))) == _lib.CVN_OK


def op_supported(x, x0, weight, scale) -> bool:
    """Whether the library's operator path serves this call (its table and scratch queries are
    non-zero for the geometry); shapes it does not serve go to the PyTorch composition.  Malformed
    arguments also answer False here and are then rejected by the composition's checks."""
    if x.dim() != 4 or x0.dim() != 4 or weight.dim() != 4:
        return False
    s = int(scale)
    B, C, h, w = (int(v) for v in x.shape)
    if s < 1 or tuple(x0.shape) != (B, C, h * s, w * s) or weight.shape[0] != 1 or weight.shape[1] != C:
        return False
    if B == 0:
        return True  # an empty batch returns its empty output without a launch (converse2d_op)
    if (s == 1 and x0.data_ptr() == x.data_ptr() and x0.stride() == x.stride() and B > 0
            and supported(x, weight, 1, 0)):
        return True  # served by the module route on the padded plane (converse2d_op)
    lib = _lib.load()
    kh, kw = int(weight.shape[2]), int(weight.shape[3])
    return (lib.cvn_converse2d_op_table_bytes(C, h, w, kh, kw, s) > 0
            and lib.cvn_converse2d_op_scratch_bytes(B, C, h, w, s) > 0)


def converse2d_backward(grad_out, x, weight, bias, scale=1, padding=2, padding_mode="circular", eps=1e-5,
                        need_x=True, need_weight=True, need_bias=True):
    """Gradients of Converse2D.forward (util_converse.py:142-192) in one library call: returns
    (grad_x, grad_weight, grad_bias), None where not requested.  grad_out (B,C,H*s,W*s); weight
    (1 or B, C, kh, kw); bias (1,C,1,1) or (C,)."""
    lib = _lib.load()
    _need_hip(grad_out, x, weight, bias)
    B, C, H, W = x.shape
    s, p = int(scale), int(padding)
    if tuple(grad_out.shape) != (B, C, H * s, W * s):
        raise RuntimeError("grad_out must be (B,C,H*scale,W*scale)")
    if weight.dim() != 4 or weight.shape[1] != C or weight.shape[0] not in (1, B):
        raise RuntimeError("weight must be (1,C,kh,kw) or (B,C,kh,kw)")
    if padding_mode not in _lib.PAD_MODES:
        raise ValueError(f"unknown padding_mode {padding_mode!r}")
    kh, kw = int(weight.shape[2]), int(weight.shape[3])
    pb = int(weight.shape[0])
    dev = x.device
    go = grad_out.contiguous()
    xc = x.contiguous()
    wc = weight.contiguous()
    bc = bias.contiguous()
    gx = torch.empty((B, C, H, W), dtype=torch.float32, device=dev) if need_x else None
    gw = torch.empty((pb, C, kh, kw), dtype=torch.float32, device=dev) if need_weight else None
    gb = torch.empty((C,), dtype=torch.float32, device=dev) if need_bias else None
    if B == 0 or not (need_x or need_weight or need_bias):
        for t in (gw, gb):
            if t is not None:
                t.zero_()
        return gx, gw, gb.reshape(bias.shape) if gb is not None else None
    nb = lib.cvn_converse2d_bwd_workspace(B, C, H, W, pb, kh, kw, s, p)
    if nb == 0:
        _lib.check(_lib.CVN_ERR_ARG, "converse2d_backward")
    ws = _workspace(dev, nb)
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    rc = lib.cvn_converse2d_bwd_f32(go.data_ptr(), xc.data_ptr(), B, C, H, W, wc.data_ptr(), pb, kh, kw,
                                    bc.data_ptr(), float(eps), s, p, _lib.PAD_MODES[padding_mode], ptr(gx), ptr(gw),
                                    ptr(gb), ws.data_ptr(), nb, _stream(dev))
    _lib.check(rc, "converse2d_backward")
    return gx, gw, gb.reshape(bias.shape) if gb is not None else None


class Converse2DFunction(torch.autograd.Function):
    """Converse2D.forward with the library's forward and backward kernels (the reference gets its
    gradients from autograd through the composite op, converse2d.cpp:223-227)."""

    @staticmethod
    def forward(ctx, x, weight, bias, scale, padding, padding_mode, eps):
        ctx.save_for_backward(x, weight, bias)
        ctx.cfg = (scale, padding, padding_mode, eps)
        # the parameters change between training steps, so their tables are not cached
        return converse2d_fused(x, weight, bias.reshape(-1), scale, padding, padding_mode, eps, cache=False)

    @staticmethod
    def backward(ctx, grad_out):
        x, weight, bias = ctx.saved_tensors
        s, p, mode, eps = ctx.cfg
        nx, nw, nb = ctx.needs_input_grad[:3]
        gx, gw, gb = converse2d_backward(grad_out, x, weight, bias, s, p, mode, eps, nx, nw, nb)
        return gx, gw, gb, None, None, None, None


def converse2d_train(x, weight, bias, scale=1, padding=2, padding_mode="circular", eps=1e-5):
    """Differentiable Converse2D forward on the HIP kernels (forward and backward)."""
    return Converse2DFunction.apply(x, weight, bias, scale, padding, padding_mode, eps)


def converse2d_op(x, x0, weight, bias, scale, eps=1e-5, cache=True):
    """The reference op (converse2d.cpp:165-209): x padded (B,C,h,w), x0 (B,C,h*s,w*s) arbitrary;
    returns the uncropped (B,C,h*s,w*s) solution.  The op table (OTF and alias-class terms) is cached
    per (psf, bias, eps, geometry) like the reference's OTF (p2o_cached, converse2d.cpp:58-102)."""
    lib = _lib.load()
    composite.check_op_args(x, x0, weight, bias, scale)
    s = int(scale)
    _need_hip(x, x0, weight, bias)
    B, C, h, w = x.shape
    if tuple(x0.shape) != (B, C, h * s, w * s) or weight.shape[1] != C or bias.shape[1] != C:
        raise RuntimeError("shape mismatch between x, x0, weight and bias")
    if (s == 1 and x0.data_ptr() == x.data_ptr() and x0.stride() == x.stride() and B > 0
            and supported(x, weight, 1, 0)):
        # x0 is x, as the reference module passes it at scale 1 (util_converse.py:166): then
        # X0 = Y and the solve is the module's X = Y (conj K + lambda) / (|K|^2 + lambda) on the
        # given (already padded) plane, one forward and one inverse transform instead of two and one
        return converse2d_fused(x, weight, bias.reshape(-1), 1, 0, "constant", eps, cache=cache)
    x, x0 = x.contiguous(), x0.contiguous()
    dev = x.device
    out = torch.empty((B, C, h * s, w * s), dtype=torch.float32, device=dev)
    if B == 0:
        return out
    kh, kw = int(weight.shape[2]), int(weight.shape[3])
    tb = lib.cvn_converse2d_op_table_bytes(C, h, w, kh, kw, s)
    sb = lib.cvn_converse2d_op_scratch_bytes(B, C, h, w, s)
    if tb == 0 or sb == 0:
        _lib.check(lib.cvn_converse2d_op_f32(None, None, B, C, h, w, None, kh, kw, None, float(eps), s, None, None,
                                             0, None), "converse2d_op")
    st = _stream(dev)
    key = None
    table = None
    if cache and cacheable(weight, bias):
        key = _cache_key("op", weight, bias, eps, (C, h, w, kh, kw, s), 0, dev)
        table = table_cache.get(key)
    if table is None:
        wc, bc = weight.contiguous(), bias.contiguous()
        table = torch.empty(tb, dtype=torch.uint8, device=dev)
        _lib.check(lib.cvn_converse2d_op_table_f32(wc.data_ptr(), kh, kw, bc.data_ptr(), float(eps), C, h, w, s,
                                                   table.data_ptr(), tb, st), "converse2d op table")
        if key is not None:
            table_cache.put(key, table, (weight, bias))
    ws = _workspace(dev, sb)
    rc = lib.cvn_converse2d_op_apply_f32(x.data_ptr(), x0.data_ptr(), B, C, h, w, s, table.data_ptr(), tb,
                                         ws.data_ptr(), sb, out.data_ptr(), st)
    _lib.check(rc, "converse2d_op")
    return out


def converse2d_fwd_oneshot(x, weight, bias, scale=1, padding=2, padding_mode="circular", eps=1e-5, act=None):
    """cvn_converse2d_fwd_f32: the whole module-level forward (table and apply) in one library call, on
    the route the library picks, with one caller workspace."""
    lib = _lib.load()
    _need_hip(x, weight, bias)
    B, C, H, W = x.shape
    s, p = int(scale), int(padding)
    kh, kw, pb = int(weight.shape[2]), int(weight.shape[3]), int(weight.shape[0])
    x, wc, bc = x.contiguous(), weight.contiguous(), bias.contiguous()
    if x.data_ptr() % 16:  # the fused route reads rows as 16-byte vectors
        x = x.clone()
    out = torch.empty((B, C, H * s, W * s), dtype=torch.float32, device=x.device)
    nb = lib.cvn_converse2d_fwd_workspace(B, C, H, W, pb, kh, kw, s, p)
    ws = _workspace(x.device, max(nb, 1))
    rc = lib.cvn_converse2d_fwd_f32(x.data_ptr(), B, C, H, W, wc.data_ptr(), pb, kh, kw, bc.data_ptr(), float(eps), s,
                                    p, _lib.PAD_MODES[padding_mode], _lib.ACT_GELU if act == "gelu" else _lib.ACT_NONE,
                                    out.data_ptr(), ws.data_ptr(), nb, _stream(x.device))
    _lib.check(rc, "converse2d_fwd")
    return out


def layernorm_cf(x, weight, bias, eps):
    """LayerNorm(data_format='channels_first') (util_converse.py:63-68)."""
    lib = _lib.load()
    _need_hip(x, weight, bias)
    x = x.contiguous()
    B, C = x.shape[:2]
    HW = x[0, 0].numel() if B > 0 else 0
    y = torch.empty_like(x)
    _lib.check(lib.cvn_layernorm_cf_f32(x.data_ptr(), B, C, HW, weight.contiguous().data_ptr(),
                                        bias.contiguous().data_ptr(), float(eps), y.data_ptr(),
                                        _stream(x.device)), "layernorm_cf")
    return y


def _wmat(weight):
    return weight.reshape(weight.shape[0], -1).contiguous()


def conv1x1(x, weight, bias=None, act=None, residual=None, res_scale=None, ln=None, out=None):
    """act(W x + b) [then res_scale * . + residual]; nn.Conv2d(cin, cout, 1) semantics.
    ln=(ln_weight, ln_bias, eps) applies channels-first LayerNorm to x first (fused prologue)."""
    lib = _lib.load()
    _need_hip(x, weight, bias, residual, res_scale)
    x = x.contiguous()
    B, Cin, H, W = x.shape
    Wm = _wmat(weight)
    Cout = Wm.shape[0]
    if Wm.shape[1] != Cin:
        raise RuntimeError("weight does not match input channels")
    y = out if out is not None else torch.empty((B, Cout, H, W), dtype=torch.float32, device=x.device)
    if residual is not None:
        residual = residual.contiguous()
    bptr = bias.contiguous().data_ptr() if bias is not None else None
    rptr = residual.data_ptr() if residual is not None else None
    sptr = res_scale.contiguous().data_ptr() if res_scale is not None else None
    a = _lib.ACT_GELU if act == "gelu" else _lib.ACT_NONE
    st = _stream(x.device)
    if ln is None:
        rc = lib.cvn_conv1x1_f32(x.data_ptr(), B, Cin, H * W, Wm.data_ptr(), bptr, Cout, a, rptr, sptr,
                                 y.data_ptr(), st)
    else:
        lw, lb, leps = ln
        rc = lib.cvn_ln_conv1x1_f32(x.data_ptr(), B, Cin, H * W, lw.contiguous().data_ptr(),
                                    lb.contiguous().data_ptr(), float(leps), Wm.data_ptr(), bptr, Cout, a, rptr,
                                    sptr, y.data_ptr(), st)
    _lib.check(rc, "conv1x1")
    return y


def ln_mlp_residual(x, ln_w, ln_b, ln_eps, w1, b1, w2, b2, res_scale=None, out=None):
    """x + res_scale * (W2 GELU(W1 LN(x) + b1) + b2): ConverseBlock.conv2 plus its residual."""
    lib = _lib.load()
    _need_hip(x, w1, b1, w2, b2, res_scale)
    x = x.contiguous()
    B, C, H, W = x.shape
    W1 = _wmat(w1)
    W2 = _wmat(w2)
    y = out if out is not None else torch.empty_like(x)
    rc = lib.cvn_ln_mlp_residual_f32(x.data_ptr(), B, C, H * W, ln_w.contiguous().data_ptr(),
                                     ln_b.contiguous().data_ptr(), float(ln_eps), W1.data_ptr(),
                                     b1.contiguous().data_ptr(), W1.shape[0], W2.data_ptr(),
                                     b2.contiguous().data_ptr(),
                                     res_scale.contiguous().data_ptr() if res_scale is not None else None,
                                     y.data_ptr(), _stream(x.device))
    _lib.check(rc, "ln_mlp_residual")
    return y


TAIL_SHAPES = {(128, 64, 128)}  # (Ct, C, Cmid) of cvn_conv_ln_mlp_residual_f32


def conv_ln_mlp_residual(t, x, w0, b0, ln_w, ln_b, ln_eps, w1, b1, w2, b2, res_scale1=None, res_scale2=None,
                         out=None, head=None, t_act=None):
    """ConverseBlock tail: y' = x + res_scale1 (W0 a(t) + b0); y = y' + res_scale2 (W2 GELU(W1 LN(y') + b1) + b2),
    a(t) = GELU(t) for t_act='gelu' (t the Converse2D output before the block's GELU), else t.
    With head = (ln_w, ln_b, ln_eps, w, b) of the next block, also returns its Converse2D input
    GELU(w LN(y) + b): (y, t_next); otherwise y."""
    lib = _lib.load()
    _need_hip(t, x, w0, b0, w1, b1, w2, b2, res_scale1, res_scale2)
    t = t.contiguous()
    x = x.contiguous()
    B, Ct, H, W = t.shape
    C = x.shape[1]
    W0, W1, W2 = _wmat(w0), _wmat(w1), _wmat(w2)
    y = out if out is not None else torch.empty_like(x)
    ptr = lambda v: v.contiguous().data_ptr() if v is not None else None
    act = _lib.ACT_GELU if t_act == "gelu" else _lib.ACT_NONE
    common = (t.data_ptr(), act, B, Ct, H * W, W0.data_ptr(), ptr(b0), ptr(res_scale1), x.data_ptr(), C, ptr(ln_w),
              ptr(ln_b), float(ln_eps), W1.data_ptr(), ptr(b1), W1.shape[0], W2.data_ptr(), ptr(b2), ptr(res_scale2),
              y.data_ptr())
    if head is None:
        _lib.check(lib.cvn_conv_ln_mlp_residual_f32(*common, _stream(x.device)), "conv_ln_mlp_residual")
        return y
    hw, hb, heps, wh, bh = head
    _need_hip(wh, bh)
    Wh = _wmat(wh)
    tn = torch.empty((B, Wh.shape[0], H, W), device=x.device, dtype=x.dtype)
    _lib.check(lib.cvn_conv_ln_mlp_head_f32(*common, ptr(hw), ptr(hb), float(heps), Wh.data_ptr(), ptr(bh),
                                            tn.data_ptr(), _stream(x.device)), "conv_ln_mlp_head")
    return y, tn


def copy_(dst, src):
    """Plain device copy through the library (HBM calibration kernel)."""
    lib = _lib.load()
    _need_hip(dst, src)
    _lib.check(lib.cvn_copy_f32(src.data_ptr(), dst.data_ptr(), src.numel(), _stream(src.device)), "copy")
    return dst
