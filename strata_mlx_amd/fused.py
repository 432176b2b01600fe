"""Either side of the expert path: the router, its choice of experts and the combine; strata_mlx/fused.py:334-497
with torch tensors on the GPU in place of mx.array.

    WindowLinear  a float16 linear layer (the router) whose products come back in float32, read as it is
    top_k         the k largest logits of each row, ties to the lower index; with `weights`, their softmax
    moe_combine   sum_k y_k * w_k plus sigmoid(g) * the shared expert, in the reference's order and rounding
    route         router -> top_k -> softmax, as _Routed.__call__ makes the experts' indices and weights
    RoutedMoE     the whole MoE block of _Routed.__call__: route, the routed experts, the shared expert and its
                  gate, moe_combine; at one token the shared expert rides in the routed launches
"""

import torch

from . import _lib

COMBINE_UPTO = 16  # tokens; strata_mlx/fused.py:468


class WindowLinear:
    """A float16 `nn.Linear` without bias whose products come back in float32; strata_mlx/fused.py:356-390.
    Up to `upto` tokens of float16 / float32 activations go through the kernel, longer inputs through torch."""

    upto = 8

    def __init__(self, weight: torch.Tensor):
        if weight.dtype != torch.float16 or weight.ndim != 2:
            raise ValueError("WindowLinear takes a float16 (rows, cols) weight")
        _lib.require_device(weight)
        self.weight = weight.contiguous()
        self.rows, self.cols = weight.shape

    def takes(self, x: torch.Tensor) -> bool:
        return x.numel() // self.cols <= self.upto and x.dtype in (torch.float16, torch.float32) and self.cols % 8 == 0

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if not self.takes(x):
            return x.float() @ self.weight.float().T
        tokens = x.numel() // self.cols
        x2 = x.reshape(tokens, self.cols).contiguous()
        out = torch.empty((tokens, self.rows), dtype=torch.float32, device=x.device)
        _lib.check(_lib.library().strata_router_matvec(self.weight.data_ptr(), self.rows, self.cols, x2.data_ptr(),
                                                         tokens, _lib.dtype_id(x.dtype), out.data_ptr(),
                                                         _lib.stream()), "router")
        return out.reshape(*x.shape[:-1], self.rows)


def top_k(logits: torch.Tensor, k: int, weights: bool = False):
    """The indices of the k largest logits (..., N) float32, largest first, ties to the lower index: the order
    `mx.argpartition(-logits, k - 1)[..., :k]` gives (strata_mlx/fused.py:422-436). With `weights`, also the
    softmax of those logits (float32), as _Routed.__call__ takes it (fused.py:490-491)."""
    n = logits.shape[-1]
    if logits.dtype != torch.float32:
        raise ValueError("top_k takes float32 logits")
    rows = logits.numel() // n
    lg = logits.reshape(rows, n).contiguous()
    idx = torch.empty((rows, k), dtype=torch.int32, device=logits.device)
    w = torch.empty((rows, k), dtype=torch.float32, device=logits.device) if weights else None
    _lib.check(_lib.library().strata_top_k(lg.data_ptr(), rows, n, k, idx.data_ptr(), _lib.ptr(w), _lib.stream()),
               "top_k")
    idx = idx.reshape(*logits.shape[:-1], k)
    return (idx, w.reshape(*logits.shape[:-1], k)) if weights else idx


def moe_combine(y: torch.Tensor, w: torch.Tensor, g: torch.Tensor, s: torch.Tensor) -> torch.Tensor | None:
    """y (..., K, D) half, w (..., K) float32, g (..., 1) half, s (..., D) half -> (..., D), or None where the
    reference's kernel does not take it (strata_mlx/fused.py:471-481)."""
    *lead, k, d = y.shape
    rows = y.numel() // (k * d)
    if rows > COMBINE_UPTO or y.dtype != torch.float16 or w.dtype != torch.float32 or d % 256:
        return None
    out = torch.empty((rows, d), dtype=y.dtype, device=y.device)
    yy, ww = y.reshape(rows, k, d).contiguous(), w.reshape(rows, k).contiguous()
    gg, ss = g.reshape(rows).to(torch.float16).contiguous(), s.reshape(rows, d).to(torch.float16).contiguous()
    _lib.check(_lib.library().strata_moe_combine(yy.data_ptr(), ww.data_ptr(), gg.data_ptr(), ss.data_ptr(), rows, k,
                                                 d, _lib.dtype_id(y.dtype), out.data_ptr(), _lib.stream()),
               "moe_combine")
    return out.reshape(*lead, d)


def route(router: WindowLinear, x: torch.Tensor, k: int):
    """The experts of each token and their weights: (indices (..., k) int32, weights (..., k) float32), as
    strata_mlx/fused.py:488-491 makes them."""
    logits = router(x)
    return top_k(logits, k, weights=True)


_route_counts = {}


def _route_count(device: torch.device) -> torch.Tensor:
    """The count strata_router_route keeps for one device and stream, zeroed when first made (each launch leaves
    it at zero)."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    c = _route_counts.get(key)
    if c is None:
        c = torch.zeros(1, dtype=torch.int32, device=device)
        _route_counts[key] = c
    return c


def route_gated(router: WindowLinear, x: torch.Tensor, experts: int, k: int):
    """route() and the rows of the router's weight past the experts' (a shared expert's gate, stacked under the
    router's rows) in one launch (strata_router_route): (indices (tokens, k) int32, weights (tokens, k) float32,
    those rows' products (tokens, rows - experts) float16), or None where the launch does not take the case (more
    than 8 tokens, a float type other than float16 / float32); the caller then makes the calls apart."""
    x2 = x.reshape(-1, router.cols).contiguous()
    tokens = x2.shape[0]
    if tokens == 0 or tokens > 8 or x2.dtype not in (torch.float16, torch.float32) or router.cols % 8:
        return None
    dev = x.device
    logits = torch.empty((tokens, router.rows), dtype=torch.float32, device=dev)
    idx = torch.empty((tokens, k), dtype=torch.int32, device=dev)
    w = torch.empty((tokens, k), dtype=torch.float32, device=dev)
    nx = router.rows - experts
    extra = torch.empty((tokens, nx), dtype=torch.float16, device=dev) if nx > 0 else None
    rc = _lib.library().strata_router_route(router.weight.data_ptr(), router.rows, router.cols, x2.data_ptr(), tokens,
                                            _lib.dtype_id(x2.dtype), logits.data_ptr(), experts, k, idx.data_ptr(),
                                            w.data_ptr(), _lib.ptr(extra), _route_count(dev).data_ptr(), _lib.stream())
    if rc == _lib.ERR_SHAPE:
        return None
    _lib.check(rc, "router_route")
    return idx, w, extra


class RoutedMoE:
    """The model's MoE block with the router's choice made by `top_k` and its end by `moe_combine`
    (strata_mlx/fused.py:484-497, `_Routed.__call__`): the router's logits, the top_k experts and the softmax of
    their logits (`route`); y = the routed experts (`switch`, a blocks.BlockSwitchGLU); g = shared_expert_gate(x) (a
    WindowLinear of one row); s = the shared expert, down . swiglu(gate . x, up . x) (dense.BlockLinear layers of the
    file's blocks); then moe_combine(y, w, g, s), or where it declines, sum_k y_k * w_k in float32 rounded to x's
    type, plus sigmoid(g) * s, in float32 as MLX promotes it.

    At one token the router's rows and the shared expert's gate go through one launch (their products), the routed
    gate/up launch makes the choice of experts from those logits and takes the shared expert's gate and up with its
    own rows (blocks.moe_gate_up_swiglu_shared), and the routed down launch takes the shared expert's down
    (blocks.expert_matvec_shared): four launches with the combine. Where a launch declines, the choice comes from
    the router's own launch (route_gated) or the calls run apart. `last_path` says which ran."""

    def __init__(self, router: WindowLinear, switch, shared_gate, shared_up, shared_down,
                 shared_expert_gate: WindowLinear, k: int):
        self.router, self.switch, self.k = router, switch, k
        self.shared_gate, self.shared_up, self.shared_down = shared_gate, shared_up, shared_down
        self.shared_expert_gate = shared_expert_gate
        self.last_path = None
        # the router's rows and the shared expert's gate as one weight: its products and the choice in one launch
        self.stacked = None
        if shared_expert_gate.cols == router.cols:
            self.stacked = WindowLinear(torch.cat([router.weight, shared_expert_gate.weight]))

    def shared_expert(self, x: torch.Tensor) -> torch.Tensor:
        """down . swiglu(gate . x, up . x) of the shared expert, its own launches: (tokens, hidden)."""
        from . import dense
        _, _, h = dense.gate_up_swiglu(self.shared_gate, self.shared_up, x)
        return self.shared_down(h)

    def _routed_choice(self, x: torch.Tensor):
        """At one token: the router's products (the stacked weight), then the gate/up launch that makes the choice
        of experts itself: (y (1, k, hidden), s (1, hidden), idx, w, g) or None."""
        from . import blocks
        if self.stacked is None or x.shape[0] != 1 or not self.stacked.takes(x):
            return None
        sw = self.switch
        logits = self.stacked(x)
        r = blocks.moe_gate_up_swiglu_shared(sw.gate_proj, sw.up_proj, x, logits, self.router.rows, self.k,
                                             self.shared_gate, self.shared_up)
        if r is None:
            return None
        h, idx, w, sh, g = r
        y, s = self._down(idx, h, sh)
        self.last_path = "choice in the launch" + ("" if self.last_path == "riding" else ", shared down apart")
        return y, s, idx.reshape(1, self.k), w.reshape(1, self.k), g

    def _down(self, flat: torch.Tensor, h: torch.Tensor, sh: torch.Tensor):
        """The routed down with the shared expert's down in it where the launch takes it: (y (1, k, hidden), s)."""
        from . import blocks
        sw = self.switch
        both = blocks.expert_matvec_shared(sw.down_proj, flat, self.shared_down)(h, sh)
        if both is None:  # the down launch does not take it: the shared down on its own launch
            y, s = blocks.expert_matvec(sw.down_proj, flat, h), self.shared_down(sh)
            self.last_path = "gate/up riding"
        else:
            y, s = both
            self.last_path = "riding"
        return y.reshape(1, self.k, -1), s

    def _riding(self, x: torch.Tensor, idx: torch.Tensor):
        """(y (1, k, hidden), s (1, hidden)) with the shared expert in the routed launches, or None."""
        from . import blocks
        sw = self.switch
        flat = idx.reshape(-1)
        r = blocks.gate_up_swiglu_shared(sw.gate_proj, sw.up_proj, x, flat, self.shared_gate, self.shared_up)
        if r is None:
            return None
        _, _, h, sh = r
        return self._down(flat, h, sh)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        lead, hidden = x.shape[:-1], x.shape[-1]
        x2 = x.reshape(-1, hidden)
        fused = self._routed_choice(x2)
        if fused is not None:
            y, s, idx, w, g = fused
        else:
            both_gates = route_gated(self.stacked, x2, self.router.rows, self.k) if self.stacked is not None else None
            if both_gates is None:
                idx, w = route(self.router, x2, self.k)
                g = self.shared_expert_gate(x2)
            else:
                idx, w, g = both_gates
            both = self._riding(x2, idx) if x2.shape[0] == 1 else None
            if both is None:
                y, s = self.switch(x2, idx).reshape(x2.shape[0], self.k, -1), self.shared_expert(x2)
                self.last_path = "apart"
            else:
                y, s = both
        out = moe_combine(y, w, g, s)
        if out is None:
            out = (y.float() * w[..., None]).sum(dim=-2).to(x.dtype).float() + torch.sigmoid(g.float()) * s.float()
        return out.reshape(*lead, -1)
