"""HiMuon optimizer on MI355X: the reference's public surface over HIP kernels.

Drop-in for ``tang0389/himuon`` ``src/himuon/optimizers/himuon.py``: same
constructor signature and defaults (himuon.py:64-80), param-group keys,
``tile_size`` normalisation (173-179), ``reconfigure`` (188-213),
``xlayer_plan`` (407-415), plan dicts (483-586), ``_balanced_chunks``
(459-481), ``_auto_b_hw`` (376-403), graph warm-up / capture / replay state
machine (1048-1109) with LR and weight decay applied outside the graph
(215-228), and ``newton_schulz`` (263-284).

What changes is the GPU body of a step. Per bucket of same-shape tiles the
step issues one fused momentum+gather launch, one normaliser launch, the NS5
launches per chunk and one untile launch (libhimuon_hip.so, C ABI in
include/himuon_hip.h) instead of per-parameter torch/inductor/Triton ops.
Full-matrix (numel <= tile area) parameters of equal shape are batched into
one NS group instead of one NS call per parameter (himuon.py:827-876); the
math per matrix is unchanged.

There is no CPU path: ``step()`` on non-HIP tensors raises, as the
reference's does without its GPU kernels (triton_kernels/__init__.py:8-19).
FSDP bank parameters (DTensor muon parameters whose rank-local shard is a
3-D bank (N_local, H, W), himuon.py:419-457, 894-1020) take the per-bank
path: each bank's N_local matrices are tiled separately (padded per matrix),
NS runs on all of the bank's tiles in one call, and WD/LR is applied to the
local shard in place; nothing crosses ranks, so no collective runs.
"""

from __future__ import annotations

import math

import torch
from torch.optim import Optimizer

from .. import _native as nat
from ..engine import AdamwTables, ApplyTables, TileGroup, update_dtype
from ..engine import newton_schulz as _hip_newton_schulz

try:
    from torch.distributed.tensor import DTensor as _DTensor  # type: ignore
except Exception:  # pragma: no cover
    _DTensor = None  # type: ignore


class HiMuon(Optimizer):
    """Hierarchical Muon with cross-layer batched NS on HIP kernels.

    Args (identical to the reference, himuon.py:48-62):
        params: model parameters
        lr: learning rate (default 0.02)
        momentum: momentum coefficient (default 0.95)
        nesterov: use Nesterov momentum (default True)
        weight_decay: weight decay (default 0.1)
        tile_size: int -> (T, T) tiles; (Th, Tw) -> non-square tiles (default 512)
        ns_steps: Newton-Schulz iterations (default 5)
        use_muon: Muon path, otherwise AdamW fallback (default True)
        lr_adjust: "tile" (lr * 0.2 * sqrt(max block dim)) or "none"
        adamw_betas / adamw_eps: AdamW fallback hyper-parameters
        b_hw: cross-layer chunk cap (None -> from device memory)
        cuda_graph: capture the step in a hipGraph after ``cuda_graph_warmup``
            eager steps (the name is kept for drop-in compatibility).
    """

    # Muon buckets apply their WD/LR inside the untile (himuon_untile_apply)
    # when their parameters allow it; False keeps update tensors and the
    # separate WD/LR pass for every bucket (same parameters, bit for bit).
    _fuse_untile: bool = True
    # Such buckets on 128 x 128 NS tiles run the whole step (momentum to
    # WD/LR) as one LDS-resident launch per chunk (himuon_lds_step); False
    # keeps the gather / NS / untile launches (same results, bit for bit).
    _fuse_lds_step: bool = True
    # fused-untile buckets of 512 x 512 tiles: the untile with WD/LR runs
    # inside the last NS iteration (himuon_ns5_untile_apply)
    _fuse_ns_untile: bool = True
    # NS kernel family of every tile group (a key of _native.NS_FAMILIES):
    # "auto", the per-geometry choice; the others are comparison runs, which
    # also keep 128 x 128 buckets off the one-launch LDS step for "block128".
    _ns_family: str = "auto"

    def __init__(
        self,
        params,
        lr=0.02,
        momentum=0.95,
        nesterov=True,
        weight_decay=0.1,
        tile_size=512,
        ns_steps=5,
        use_muon=True,
        lr_adjust="tile",
        adamw_betas=(0.95, 0.95),
        adamw_eps=1e-8,
        b_hw=None,
        cuda_graph=True,
        cuda_graph_warmup=3,
    ):
        tile_size = self._normalize_defaults(tile_size)
        defaults = dict(
            lr=lr,
            momentum=momentum,
            nesterov=nesterov,
            weight_decay=weight_decay,
            tile_size=tile_size,
            ns_steps=ns_steps,
            use_muon=use_muon,
            adamw_betas=adamw_betas,
            adamw_eps=adamw_eps,
        )
        super().__init__(params, defaults)

        self._b_hw_override = b_hw
        self._memory_budget_fraction = 0.15
        # bucket_key -> bf16 NS tile buffer (n_tiles, mp, np) of that bucket.
        self._concat_buffers: dict[tuple, torch.Tensor] = {}
        self._cached_plan: "list[dict] | None" = None
        self._last_step_stats: dict = {"ns_gpu_ms": 0.0, "ns_launches": 0, "total_B": 0, "avg_batch": 0.0}

        self._cuda_graph_enabled = bool(cuda_graph)
        self._cuda_graph_warmup = int(cuda_graph_warmup)
        self._cuda_graph: "torch.cuda.CUDAGraph | None" = None
        self._graph_step_count: int = 0
        self._in_graph_region: bool = False
        # (param, update_tensor, group_idx), filled at capture, applied after replay.
        self._pending_updates: list[tuple] = []
        self._apply_tables: "ApplyTables | None" = None  # device tables for _pending_updates
        # Fused AdamW fallback: persistent update buffers and device tables,
        # rebuilt when the set of (param, grad storage) changes.
        # Device (scale, alpha) per param group, written before each step and
        # read by the fused untile+WD/LR kernel (also during graph replay).
        self._lrwd: "torch.Tensor | None" = None
        self._adamw_updates: dict = {}
        self._adamw_tables: "AdamwTables | None" = None
        self._adamw_sig: "tuple | None" = None

        # Device state of the HIP path, rebuilt after reconfigure().
        self._groups: "list[dict] | None" = None  # tiled buckets + full-NS shape groups
        self._workspace: "torch.Tensor | None" = None
        # (param, param storage) of every parameter with a grad when the
        # device state (plan, tile groups, graph) was built, and where those
        # grads lived when the graph was captured.
        self._state_sig: "tuple | None" = None
        self._grad_sig: "tuple | None" = None

        if lr_adjust not in ("none", "tile"):
            raise ValueError(f"lr_adjust must be 'none' or 'tile', got {lr_adjust!r}")
        self.lr_adjust = lr_adjust

    # -- Reconfiguration (himuon.py:173-228) --------------------------------

    @staticmethod
    def _normalize_defaults(tile_size):
        if isinstance(tile_size, int):
            tile_size = (tile_size, tile_size)
        tile_size = tuple(tile_size)
        assert len(tile_size) == 2 and all(t > 0 for t in tile_size)
        return tile_size

    def adjust_lr_for_muon(self, lr, block_shape):
        """Adapted from Muon's adjust_lr_for_muon."""
        if self.lr_adjust == "none":
            return lr
        a, b = block_shape[:2]
        return lr * 0.2 * math.sqrt(max(a, b))

    def reconfigure(self, **updates):
        """Update param-group defaults mid-training (e.g., tile_size) and drop
        the cached plan, buffers and captured graph."""
        for group in self.param_groups:
            ts = self._normalize_defaults(updates.get("tile_size", group["tile_size"]))
            for k, v in updates.items():
                if k in group:
                    group[k] = v
            if "tile_size" in updates:
                group["tile_size"] = ts
        self._invalidate_plan_cache()

    def _invalidate_plan_cache(self):
        """Flush plan, tile buffers, device state, graph and pending updates.
        (The reference also resets torch._dynamo for its compiled helpers; this
        path compiles nothing at run time.)"""
        self._concat_buffers.clear()
        self._cached_plan = None
        self._groups = None
        self._workspace = None
        self._drop_graph()
        self._adamw_tables = None
        self._adamw_sig = None

    def _local(self, t: torch.Tensor) -> torch.Tensor:
        """The rank-local tensor of a DTensor (shares its storage), else t."""
        return t.to_local() if self._is_dtensor(t) else t

    def _storage_sig(self) -> tuple[tuple, tuple]:
        """(which parameters have a grad and where each such parameter's
        storage lives, where each of those grads lives), for the local shard of
        DTensors. The plan and tile groups depend on the first; the descriptor
        tables and a captured graph hold pointers of both."""
        with_grad = [p for g in self.param_groups for p in g["params"] if p.grad is not None]
        return (
            tuple((id(p), self._local(p).data_ptr()) for p in with_grad),
            tuple(self._local(p.grad).data_ptr() for p in with_grad),
        )

    def _drop_graph(self) -> None:
        """Forget the captured graph (the next steps warm up and recapture);
        the plan, tile groups and buffers stay."""
        self._cuda_graph = None
        self._graph_step_count = 0
        self._pending_updates.clear()
        self._apply_tables = None

    def _check_storage(self) -> None:
        """When the set of parameters with grads or the storage of any of
        them changed since the device state was built, drop the plan, device
        state and graph (the next steps warm up and recapture, as after
        reconfigure; momentum and AdamW state are kept). When only grads moved
        (zero_grad(set_to_none=True) between steps), keep the plan and tile
        groups: eager steps rewrite their descriptor tables in place (bind()),
        and a captured graph, which recorded the old pointers, is dropped and
        recaptured. The reference scans the full-matrix parameters every step
        and skips those without a grad (himuon.py:846-858) and reads p.data at
        every update (himuon.py:222-228, 343-348)."""
        struct, grads = self._storage_sig()
        if struct != self._state_sig:
            if self._state_sig is not None:
                self._invalidate_plan_cache()
            self._state_sig = struct
        elif grads != self._grad_sig and self._cuda_graph is not None:
            self._drop_graph()
        self._grad_sig = grads

    def _scale_alpha(self) -> list[float]:
        """(1 - lr*wd, -lr) per param group: the two factors of p.mul_(1 - lr*wd);
        p.add_(u, alpha=-lr) (himuon.py:222-228, 345-348); 1.0 when wd == 0."""
        out = []
        for group in self.param_groups:
            lr, weight_decay = group["lr"], group["weight_decay"]
            out += [1 - lr * weight_decay if weight_decay > 0.0 else 1.0, -lr]
        return out

    def _write_lrwd(self, device) -> None:
        """Current (scale, alpha) of every group into the device table the fused
        untile reads: one small kernel on the current stream, ordered after the
        previous replay (which may still read the table) and before this step's
        body or replay, without a host synchronisation. Groups beyond what the
        table holds are never fused (their buckets take the outside-graph
        WD/LR), so only the first APPLY_MAX_GROUPS are written."""
        vals = self._scale_alpha()[: 2 * nat.APPLY_MAX_GROUPS]
        if self._lrwd is None or self._lrwd.device != device:
            self._lrwd = torch.zeros(2 * nat.APPLY_MAX_GROUPS, device=device, dtype=torch.float32)
        nat.write_scale_alpha(self._lrwd, vals[0::2], vals[1::2])

    def _apply_pending_updates(self):
        """WD + LR application after replay, reading the current group lr/wd:
        one multi-tensor HIP launch per dtype pair (himuon_apply_updates) with
        lr/wd passed as host scalars, so schedules need no recapture. Entries
        without an update tensor belong to fused groups, whose WD/LR the untile
        already applied inside the graph."""
        if not self._pending_updates:
            return
        if self._apply_tables is None:
            todo = [e for e in self._pending_updates if e[1] is not None]
            if not todo:
                return
            self._apply_tables = ApplyTables(todo)
        scales, alphas = [], []
        for group in self.param_groups:
            lr, weight_decay = group["lr"], group["weight_decay"]
            scales.append(1 - lr * weight_decay if weight_decay > 0.0 else 1.0)
            alphas.append(-lr)
        self._apply_tables.run(scales, alphas)
        for p, update, group_idx in self._apply_tables.fallback:
            group = self.param_groups[group_idx]
            lr = group["lr"]
            weight_decay = group["weight_decay"]
            if weight_decay > 0.0:
                p.data.mul_(1 - lr * weight_decay)
            p.data.add_(update, alpha=-lr)

    # -- Newton-Schulz --------------------------------------------------------

    @staticmethod
    def newton_schulz(G, steps=5):
        """Quintic NS of G (..., M, N) on the HIP kernels; returns G's shape and
        dtype (himuon.py:263-284). ``steps`` is honoured for every shape."""
        return _hip_newton_schulz(G, steps=steps)

    # -- Tiling helpers (himuon.py:288-310), torch views only ---------------

    @staticmethod
    def _tile(tensor, tile_size):
        """Tile (H, W) -> (R, C, Th, Tw) with zero-padding."""
        tile_h, tile_w = tile_size
        h, w = tensor.shape
        pad_h = (tile_h - h % tile_h) % tile_h
        pad_w = (tile_w - w % tile_w) % tile_w
        if pad_h or pad_w:
            tensor = torch.nn.functional.pad(tensor, (0, pad_w, 0, pad_h))
        H, W = tensor.shape
        R, C = H // tile_h, W // tile_w
        return tensor.view(R, tile_h, C, tile_w).permute(0, 2, 1, 3).contiguous(), (h, w, pad_h, pad_w)

    @staticmethod
    def _untile(tiled, info):
        """Restore (R, C, Th, Tw) -> (H, W) and remove padding."""
        h, w, pad_h, pad_w = info
        R, C, Th, Tw = tiled.shape
        restored = tiled.permute(0, 2, 1, 3).contiguous().view(R * Th, C * Tw)
        return restored[:h, :w] if (pad_h or pad_w) else restored

    # -- AdamW fallback (himuon.py:359-372, 878-888) --------------------------

    def _compute_adamw_step(self, p, g, betas, eps):
        if "step" not in self.state[p]:
            self.state[p]["step"] = torch.zeros((), device=g.device)
            self.state[p]["moment1"] = torch.zeros_like(g)
            self.state[p]["moment2"] = torch.zeros_like(g)
        step = self.state[p]["step"]
        step.add_(1)
        buf1, buf2 = self.state[p]["moment1"], self.state[p]["moment2"]
        buf1.lerp_(g, 1 - betas[0])
        buf2.lerp_(g.square(), 1 - betas[1])
        bc1 = 1 - betas[0] ** step
        bc2 = 1 - betas[1] ** step
        return (buf1 / bc1) / (buf2.sqrt() / bc2**0.5 + eps)

    def _apply_wd_and_update(self, p, update, weight_decay, lr, group_idx, scaled=False):
        """Graph region: defer to _apply_pending_updates. Eager: apply now.
        ``update`` from the HIP path already carries the lr-adjust scale."""
        if self._in_graph_region:
            self._pending_updates.append((p, update, group_idx))
        else:
            if weight_decay > 0.0:
                p.data.mul_(1 - lr * weight_decay)
            p.data.add_(update, alpha=-lr)

    def _step_adamw(self, group, group_idx):
        """The reference's per-parameter torch ops (himuon.py:878-888); used
        for the parameters the fused kernel cannot take."""
        lr = group["lr"]
        weight_decay = group["weight_decay"]
        for p in group["params"]:
            if p.grad is None:
                continue
            update = self._compute_adamw_step(p, p.grad, group["adamw_betas"], group["adamw_eps"])
            self._apply_wd_and_update(p, update, weight_decay, lr, group_idx)

    def _prepare_adamw(self):
        """State (as the reference creates it: fp32 device step, zero moments in
        the grad dtype), persistent update buffers and the device tables of the
        fused AdamW step for every AdamW-group parameter with a grad. Runs
        outside graph capture; returns the list of (param, group_idx)."""
        params = []
        for group_idx, group in enumerate(self.param_groups):
            if group["use_muon"]:
                continue
            for p in group["params"]:
                if p.grad is None:
                    continue
                g = p.grad
                st = self.state[p]
                if "step" not in st:
                    st["step"] = torch.zeros((), device=g.device)
                    st["moment1"] = torch.zeros_like(g)
                    st["moment2"] = torch.zeros_like(g)
                u = self._adamw_updates.get(p)
                if u is None or u.shape != g.shape or u.dtype != g.dtype or u.device != g.device:
                    u = torch.empty_like(g, memory_format=torch.contiguous_format)
                    self._adamw_updates[p] = u
                params.append((p, group_idx))
        sig = tuple(
            (id(p), p.grad.data_ptr(), p.grad.dtype, self.state[p]["moment1"].data_ptr(),
             self._adamw_updates[p].data_ptr(), gi)
            for p, gi in params
        )
        if sig != self._adamw_sig:
            self._adamw_sig = sig
            entries = [
                (p.grad, self.state[p]["moment1"], self.state[p]["moment2"], self._adamw_updates[p],
                 self.state[p]["step"], gi)
                for p, gi in params
            ]
            self._adamw_tables = AdamwTables(entries) if entries else None
        return params

    def _step_adamw_groups(self):
        """AdamW fallback groups (himuon.py:1013/1034 -> 878-888): one fused
        HIP pass per grad dtype (himuon_adamw_step) computes step, moments and
        the update of every parameter; the update then takes the same WD/LR
        path as the reference's (deferred to after replay in graph mode)."""
        params = self._prepare_adamw()
        if not params:
            return
        tables = self._adamw_tables
        fallback = {e[0].data_ptr() for e in tables.fallback} if tables is not None else set()
        if tables is not None and tables.launches:
            b1 = [float(g["adamw_betas"][0]) for g in self.param_groups]
            b2 = [float(g["adamw_betas"][1]) for g in self.param_groups]
            ep = [float(g["adamw_eps"]) for g in self.param_groups]
            tables.run(b1, b2, ep)
        for p, gi in params:
            group = self.param_groups[gi]
            if p.grad.data_ptr() in fallback:
                update = self._compute_adamw_step(p, p.grad, group["adamw_betas"], group["adamw_eps"])
            else:
                update = self._adamw_updates[p]
            self._apply_wd_and_update(p, update, group["weight_decay"], group["lr"], gi)

    # -- Chunk cap and plan (himuon.py:376-415, 459-586) ---------------------

    def _auto_b_hw(self, T: int, dtype_bytes: int = 4) -> int:
        if not torch.cuda.is_available():
            user = self._b_hw_override
            return max(1, int(user)) if user is not None else 1
        device = torch.cuda.current_device()
        total_mem = torch.cuda.get_device_properties(device).total_memory
        budget = int(self._memory_budget_fraction * total_mem)
        bytes_per_tile = 4 * T * T * dtype_bytes
        mem_cap = max(1, budget // bytes_per_tile)
        if self._b_hw_override is not None:
            return max(1, min(int(self._b_hw_override), mem_cap))
        return mem_cap

    def xlayer_plan(self) -> list[dict]:
        if self._cached_plan is None:
            return []
        return list(self._cached_plan)

    def _is_dtensor(self, p) -> bool:
        return _DTensor is not None and isinstance(p, _DTensor)

    @staticmethod
    def _balanced_chunks(B_total: int, b_hw: int) -> list[int]:
        """ceil(B_total / b_hw) chunks of ceil(remaining / remaining_chunks)."""
        if B_total <= 0:
            return []
        n_chunks = math.ceil(B_total / b_hw)
        chunks: list[int] = []
        remaining = B_total
        for i in range(n_chunks):
            c = math.ceil(remaining / (n_chunks - i))
            chunks.append(c)
            remaining -= c
        return chunks

    def _plan_buckets(self) -> list[dict]:
        """Tiled buckets keyed (tile_h, tile_w, False, grad dtype) in
        param_groups/params order; params with numel <= tile area are left to
        the full-NS path (himuon.py:541-544)."""
        by_key: dict[tuple, list] = {}
        for group in self.param_groups:
            if not group["use_muon"]:
                continue
            tile_h, tile_w = group["tile_size"]
            for p in group["params"]:
                if p.grad is None:
                    continue
                if self._is_dtensor(p):
                    raise NotImplementedError(
                        "HiMuon (HIP path) runs on one GPU; FSDP/DTensor parameters are not supported"
                    )
                grad = p.grad
                if grad.numel() <= tile_h * tile_w:
                    continue
                h, w = grad.shape
                R = -(-h // tile_h)
                C = -(-w // tile_w)
                key = (tile_h, tile_w, False, grad.dtype)
                by_key.setdefault(key, []).append((p, group, R * C))

        plan: list[dict] = []
        for key, entries in by_key.items():
            tile_h, tile_w, _full_ns, _dtype = key
            T = max(tile_h, tile_w)
            dtype_bytes = torch.empty((), dtype=_dtype).element_size()
            b_hw = self._auto_b_hw(T, dtype_bytes=dtype_bytes)
            tile_count_per_param = [e[2] for e in entries]
            B_total = sum(tile_count_per_param)
            chunk_sizes = self._balanced_chunks(B_total, b_hw)
            plan.append(
                {
                    "bucket_key": key,
                    "param_ids": [id(e[0]) for e in entries],
                    "tile_count_per_param": tile_count_per_param,
                    "B_total": B_total,
                    "B_hw": b_hw,
                    "chunk_sizes": chunk_sizes,
                    "n_calls": len(chunk_sizes),
                    "_entries": entries,
                }
            )
        return plan

    def _plan_full_ns(self) -> list[dict]:
        """Full-NS parameters (numel <= tile area) grouped by (shape, dtype,
        ns_steps), in param_groups/params order."""
        by_key: dict[tuple, list] = {}
        for group in self.param_groups:
            if not group["use_muon"]:
                continue
            tile_h, tile_w = group["tile_size"]
            for p in group["params"]:
                if p.grad is None or self._is_dtensor(p):
                    continue
                if p.grad.numel() > tile_h * tile_w:
                    continue
                if p.grad.ndim != 2:
                    raise ValueError(f"HiMuon muon params must be 2-D, got {tuple(p.grad.shape)}")
                key = (tuple(p.grad.shape), p.grad.dtype, group["ns_steps"])
                by_key.setdefault(key, []).append((p, group))
        return [{"key": k, "entries": v} for k, v in by_key.items()]

    # -- Device state -----------------------------------------------------------

    def _momentum_buffer(self, p):
        """The parameter's momentum buffer (for a DTensor bank, a plain tensor
        shaped like the local grad shard, as the reference's per-bank path
        keeps it: himuon.py:350-357 called on the local grad, :906)."""
        st = self.state[p]
        if "momentum_buffer" not in st:
            st["momentum_buffer"] = torch.zeros_like(self._local(p.grad))
        return st["momentum_buffer"]

    def _build_groups(self, plan: list[dict]) -> list[dict]:
        group_to_idx = {id(g): i for i, g in enumerate(self.param_groups)}

        def fusable(params, gidx, grad_dtype) -> bool:
            # The untile applies WD/LR in place: one parameter dtype the kernels
            # take, row-major 2-D parameters, group indices inside the table.
            # fp16 parameters not with fp32 grads: the fused untile adds the
            # update through fp32; torch adds an fp32 update into fp16 with one
            # rounding, which the WD/LR pass reproduces.
            pd = {p.dtype for p in params}
            return (
                self._fuse_untile
                and len(pd) == 1 and next(iter(pd)) in nat.DTYPE_CODES
                and (next(iter(pd)) != torch.float16 or grad_dtype != torch.float32)
                and all(p.is_cuda and p.ndim == 2 and (p.stride(1) == 1 or p.shape[1] == 1) for p in params)
                and max(gidx) < nat.APPLY_MAX_GROUPS
            )

        out = []
        for bucket in plan:
            tile_h, tile_w, _f, dtype = bucket["bucket_key"]
            entries = bucket["_entries"]
            steps = {e[1]["ns_steps"] for e in entries}
            assert len(steps) <= 1, f"cross-layer NS requires a uniform ns_steps per bucket; saw {steps}"
            params = [e[0] for e in entries]
            gidx = [group_to_idx[id(e[1])] for e in entries]
            grp = TileGroup(
                params=params,
                grads=[p.grad for p in params],
                moms=[self._momentum_buffer(p) for p in params],
                tile_h=tile_h,
                tile_w=tile_w,
                upd_scales=[self.adjust_lr_for_muon(1.0, (tile_h, tile_w))] * len(params),
                mus=[e[1]["momentum"] for e in entries],
                nesterovs=[e[1]["nesterov"] for e in entries],
                device=params[0].grad.device,
                dtype=dtype,
                upd_dtype=update_dtype(params, dtype),
                apply_groups=gidx if fusable(params, gidx, dtype) else None,
                ns_family=self._ns_family,
            )
            if not (self._fuse_lds_step and grp.lds_step_ok()):
                # A bucket whose step runs in LDS (himuon_lds_step: 128 x 128
                # NS tiles) has no tile buffer at all, so it registers none:
                # its tiles exist only in LDS, one workgroup at a time.
                self._concat_buffers[bucket["bucket_key"]] = grp.tiles
            out.append(
                {
                    "tiles": grp,
                    "entries": [(p, g) for p, g, _ in entries],
                    "group_idx": [group_to_idx[id(g)] for _, g, _ in entries],
                    "steps": next(iter(steps)) if steps else 5,
                    "chunks": list(bucket["chunk_sizes"]),
                    "full": False,
                }
            )
        for fg in self._plan_full_ns():
            (h, w), dtype, steps = fg["key"]
            entries = fg["entries"]
            params = [p for p, _ in entries]
            gidx = [group_to_idx[id(g)] for _, g in entries]
            # One tile per matrix: tile = (h, w); lr scale from p.shape (himuon.py:872-874).
            grp = TileGroup(
                params=params,
                grads=[p.grad for p in params],
                moms=[self._momentum_buffer(p) for p in params],
                tile_h=h,
                tile_w=w,
                upd_scales=[self.adjust_lr_for_muon(1.0, p.shape) for p in params],
                mus=[g["momentum"] for _, g in entries],
                nesterovs=[g["nesterov"] for _, g in entries],
                device=params[0].grad.device,
                dtype=dtype,
                upd_dtype=update_dtype(params, dtype),
                apply_groups=gidx if fusable(params, gidx, dtype) else None,
                # the reference calls newton_schulz on the 2-D momentum
                # (himuon.py:861), whose third product is torch.addmm (249-253)
                round_once=True,
                ns_family=self._ns_family,
            )
            out.append(
                {
                    "tiles": grp,
                    "entries": entries,
                    "group_idx": [group_to_idx[id(g)] for _, g in entries],
                    "steps": steps,
                    "chunks": [grp.n_tiles],
                    "full": True,
                }
            )
        self._size_workspace(out)
        return out

    def _bank_sources(self, p, group):
        """Per-matrix (grads, momentum buffers, mus, nesterovs) of a bank
        parameter's local shard: 2-D views of the (N, H, W) grad and buffer."""
        gl = self._local(p.grad)
        buf = self._momentum_buffer(p)
        n = gl.shape[0]
        return [gl[i] for i in range(n)], [buf[i] for i in range(n)], [group["momentum"]] * n, [group["nesterov"]] * n

    def _build_bank_groups(self) -> list[dict]:
        """FSDP per-bank path (himuon.py:894-964): one tile group per bank
        parameter, over the N matrices of its local (N, H, W) shard. Each matrix
        is tiled and padded on its own (himuon.py:920-936); when the tile covers
        a whole matrix the bank runs NS on (N, H, W) directly with block (H, W)
        (:912-918). The untile applies WD/LR to the local shard in place. NS is
        the batched form (newton_schulz on a 3-D input): its third product
        rounds B X before adding a X."""
        group_to_idx = {id(g): i for i, g in enumerate(self.param_groups)}
        out = []
        for group in self.param_groups:
            if not group["use_muon"]:
                continue
            gi = group_to_idx[id(group)]
            for p in group["params"]:
                if p.grad is None:
                    continue
                if not self._is_dtensor(p):
                    raise RuntimeError(
                        "HiMuon FSDP path: muon param group contains a non-DTensor param. Mixed "
                        "DTensor/non-DTensor muon params are not supported. Wrap all muon-eligible "
                        "params with the same FSDP scheme."
                    )
                gl = self._local(p.grad)
                if gl.ndim != 3:
                    raise RuntimeError(
                        f"HiMuon FSDP per-bank path requires bank-wrapped 3D muon params; got local "
                        f"ndim={gl.ndim} (shape {tuple(gl.shape)}). Call wrap_with_banks() before fully_shard()."
                    )
                n, h, w = gl.shape
                tile_h, tile_w = group["tile_size"]
                block = (h, w) if (tile_h >= h and tile_w >= w) else (tile_h, tile_w)
                pl = self._local(p)
                slices = [pl[i] for i in range(n)]
                grads, moms, mus, nesterovs = self._bank_sources(p, group)
                fuse = (
                    self._fuse_untile and pl.dtype in nat.DTYPE_CODES
                    and (pl.dtype != torch.float16 or gl.dtype != torch.float32)
                    and pl.is_cuda and pl.is_contiguous() and gi < nat.APPLY_MAX_GROUPS
                )
                grp = TileGroup(
                    params=slices,
                    grads=grads,
                    moms=moms,
                    tile_h=block[0],
                    tile_w=block[1],
                    upd_scales=[self.adjust_lr_for_muon(1.0, block)] * n,
                    mus=mus,
                    nesterovs=nesterovs,
                    device=gl.device,
                    dtype=gl.dtype,
                    upd_dtype=update_dtype(slices, gl.dtype),
                    apply_groups=[gi] * n if fuse else None,
                    ns_family=self._ns_family,
                )
                out.append(
                    {
                        "tiles": grp,
                        "entries": [(sl, group) for sl in slices],
                        "group_idx": [gi] * n,
                        "steps": group["ns_steps"],
                        "chunks": [grp.n_tiles],
                        "full": False,
                        "bank": p,
                    }
                )
        self._size_workspace(out)
        return out

    def _size_workspace(self, groups: list[dict]) -> None:
        """One NS workspace shared by all groups, sized for the largest need."""
        need = 1
        for g in groups:
            grp = g["tiles"]
            g["sub_batch"] = grp.default_sub_batch()
            need = max(need, grp.workspace_bytes(g["sub_batch"]))
        device = groups[0]["tiles"].device if groups else None
        if device is not None and (self._workspace is None or self._workspace.numel() < need):
            self._workspace = torch.empty(need, device=device, dtype=torch.uint8)

    def _ensure_device_state(self):
        if self._has_dtensor_muon():  # FSDP per-bank path: no cross-layer plan
            if self._groups is None:
                self._groups = self._build_bank_groups()
            else:
                for g in self._groups:
                    g["tiles"].bind(*self._bank_sources(g["bank"], g["entries"][0][1]))
            return self._groups
        if self._cached_plan is None:
            self._cached_plan = self._plan_buckets()
            self._groups = None
        if self._groups is None:
            self._groups = self._build_groups(self._cached_plan)
        else:
            # Eager steps re-bind if grads/momentum moved or momentum settings changed.
            for g in self._groups:
                params = [p for p, _ in g["entries"]]
                g["tiles"].bind(
                    [p.grad for p in params],
                    [self._momentum_buffer(p) for p in params],
                    [grp["momentum"] for _, grp in g["entries"]],
                    [grp["nesterov"] for _, grp in g["entries"]],
                )
        return self._groups

    # -- Step body ----------------------------------------------------------------

    def _has_dtensor_muon(self) -> bool:
        for g in self.param_groups:
            if not g["use_muon"]:
                continue
            for p in g["params"]:
                if p.grad is not None and self._is_dtensor(p):
                    return True
        return False

    def _run_groups(self, groups) -> dict:
        use_events = not self._in_graph_region
        ev_pairs = []
        ns_launches = 0
        total_B = 0
        for g in groups:
            grp: TileGroup = g["tiles"]
            lds = self._fuse_lds_step and grp.lds_step_ok()
            nsu = not lds and self._fuse_ns_untile and grp.ns_untile_ok(g["steps"])
            if not lds:
                grp.gather()
            ofs = 0
            for c in g["chunks"]:
                if use_events:
                    ev0 = torch.cuda.Event(enable_timing=True)
                    ev1 = torch.cuda.Event(enable_timing=True)
                    ev0.record()
                if lds:
                    grp.lds_step(ofs, c, g["steps"], self._lrwd)
                elif nsu:
                    grp.ns_untile(ofs, c, g["steps"], self._workspace, g["sub_batch"], self._lrwd)
                else:
                    grp.ns(ofs, c, g["steps"], self._workspace, g["sub_batch"])
                if use_events:
                    ev1.record()
                    ev_pairs.append((ev0, ev1))
                ns_launches += 1
                total_B += c
                ofs += c
            if grp.fused:
                # WD/LR applied by the untile itself (or by the LDS-resident
                # step, or inside the last NS iteration), from the (scale,
                # alpha) table written before this step; the graph path still
                # lists the parameters as pending (without an update tensor).
                if not (lds or nsu):
                    grp.untile(g["steps"], self._lrwd)
                if self._in_graph_region:
                    for (p, _), gi in zip(g["entries"], g["group_idx"]):
                        self._pending_updates.append((p, None, gi))
            else:
                grp.untile(g["steps"])
                for (p, grp_dict), gi, upd in zip(g["entries"], g["group_idx"], grp.updates):
                    self._apply_wd_and_update(p, upd, grp_dict["weight_decay"], grp_dict["lr"], gi)
        ns_ms = 0.0
        if use_events and ev_pairs:
            ev_pairs[-1][1].synchronize()
            ns_ms = sum(a.elapsed_time(b) for a, b in ev_pairs)
        return {"ns_gpu_ms": ns_ms, "ns_launches": ns_launches, "total_B": total_B}

    def _step_body(self):
        """Momentum -> tile -> NS5 -> untile for every muon param (HIP), then the
        AdamW groups (torch), with WD/LR applied eagerly or deferred to after
        graph replay."""
        groups = self._ensure_device_state()
        stats = self._run_groups(groups) if groups else {"ns_gpu_ms": 0.0, "ns_launches": 0, "total_B": 0}
        for g in groups or ():
            # the launches are enqueued; the parameters hold their grads and
            # self.state the momentum buffers (a captured graph needs them in
            # place anyway, which _check_storage enforces)
            g["tiles"].release()
        self._step_adamw_groups()
        if groups and "bank" in groups[0]:
            # the FSDP path's stats (himuon.py:1013-1018): one NS launch per bank
            self._last_step_stats = {"ns_gpu_ms": 0.0, "ns_launches": len(groups), "total_B": 0, "avg_batch": 0.0}
            return
        n = stats["ns_launches"]
        self._last_step_stats = {
            "ns_gpu_ms": float(stats["ns_gpu_ms"]),
            "ns_launches": int(n),
            "total_B": int(stats["total_B"]),
            "avg_batch": float(stats["total_B"]) / float(n) if n > 0 else 0.0,
        }

    def _check_device(self):
        for g in self.param_groups:
            for p in g["params"]:
                if p.grad is not None and not p.grad.is_cuda:
                    raise RuntimeError(
                        "HiMuon (HIP path) requires parameters and grads on a ROCm device; "
                        "there is no CPU implementation of step()"
                    )

    def _capture_graph(self) -> None:
        """Capture momentum..untile into a hipGraph. The fused untile reads WD/LR
        from the device table step() rewrites before each replay; the
        remaining updates get theirs after replay."""
        self._ensure_device_state()  # allocate everything before capture
        self._prepare_adamw()
        torch.cuda.synchronize()
        self._pending_updates.clear()
        self._apply_tables = None
        self._cuda_graph = torch.cuda.CUDAGraph()
        self._in_graph_region = True
        try:
            with torch.cuda.graph(self._cuda_graph):
                self._step_body()
        finally:
            self._in_graph_region = False
        self._cuda_graph.replay()
        self._apply_pending_updates()
        torch.cuda.synchronize()

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            loss = closure()
        self._check_device()
        self._check_storage()
        dev = next((p.grad.device for g in self.param_groups for p in g["params"] if p.grad is not None), None)
        if dev is not None and dev.type == "cuda":
            self._write_lrwd(dev)
        if not self._cuda_graph_enabled or not torch.cuda.is_available():
            self._step_body()
            return loss
        if self._graph_step_count < self._cuda_graph_warmup:
            self._step_body()
            self._graph_step_count += 1
            return loss
        if self._cuda_graph is None:
            self._capture_graph()
            return loss
        self._cuda_graph.replay()
        self._apply_pending_updates()
        self._last_step_stats = {"ns_gpu_ms": 0.0, "ns_launches": 0, "total_B": 0, "avg_batch": 0.0}
        return loss
