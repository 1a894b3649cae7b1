"""Device state and launch sequence for one group of same-geometry NS tiles.

A ``TileGroup`` owns everything one bucket of the HiMuon step needs on the
device, allocated once so pointers stay stable for hipGraph capture:

* the bf16 NS tile buffers ``(n_tiles, mp, np)`` (the concat buffer of
  himuon.py:588-612, stored directly as the bf16 NS operand) that X
  ping-pongs between,
* the per-tile sum-of-squares partials and normalisers,
* the per-parameter ``update`` tensors the untile kernel writes (grad dtype,
  or the parameters' dtype when that is narrower: see ``update_dtype``),
* the device descriptor table (HimuonParamDesc[]) the gather/untile kernels read.

``run()`` issues: momentum+gather -> tile scale -> NS5 per chunk -> untile.
"""

from __future__ import annotations

import torch

from . import _native as nat


def update_dtype(params, grad_dtype: torch.dtype) -> torch.dtype:
    """Storage dtype of a group's update tensors. The update's only consumer
    is the WD/LR application, which (as torch's in-place add does) first rounds
    it to the parameter dtype; when every parameter of the group is bf16 and
    the grads are fp32, storing the update already rounded to bf16 gives the
    same parameters bit for bit and moves 2 bytes per element instead of 4.
    Not for fp16 parameters: torch adds an fp32 update into them with one
    rounding from the exact value, an fp16 update through fp32 (two), so the
    stored dtype would change the result."""
    pdts = {p.dtype for p in params}
    if grad_dtype == torch.float32 and pdts == {torch.bfloat16}:
        return torch.bfloat16
    return grad_dtype


class TileGroup:
    def __init__(
        self,
        params: list[torch.Tensor],
        grads: list[torch.Tensor],
        moms: list[torch.Tensor | None],
        tile_h: int,
        tile_w: int,
        upd_scales: list[float],
        mus: list[float],
        nesterovs: list[bool],
        device: torch.device,
        dtype: torch.dtype,
        upd_dtype: torch.dtype | None = None,
        apply_groups: list[int] | None = None,
        round_once: bool = False,
        ns_family: str = "auto",
    ):
        self.tile_h, self.tile_w = int(tile_h), int(tile_w)
        # NS kernel family (a key of _native.NS_FAMILIES): "auto" is the
        # per-geometry choice the optimizer runs; the others are comparison runs.
        if ns_family not in nat.NS_FAMILIES:
            raise ValueError(f"unknown NS kernel family {ns_family!r}")
        self.ns_family = ns_family
        # NS third product rounded once (the reference's 2-D addmm form,
        # himuon.py:249-253): full-matrix groups and 2-D newton_schulz calls.
        self.round_once = bool(round_once)
        self.m, self.n, self.mp, self.np, self.trans = nat.ns_geometry(self.tile_h, self.tile_w)
        self.device = device
        self.dtype = dtype  # grads and momentum
        # Update buffers: the grad dtype, or the parameters' own narrower dtype
        # when the only consumer of the update rounds it to that dtype first.
        self.upd_dtype = dtype if upd_dtype is None else upd_dtype
        self.params = params
        # Fused mode (apply_groups given): the untile applies each parameter's
        # group WD/LR to the parameter in place (himuon_untile_apply) and no
        # update tensors exist.
        self.fused = apply_groups is not None
        if self.fused:
            pdts = {p.dtype for p in params}
            if len(pdts) != 1:
                raise TypeError(f"fused untile needs one parameter dtype per group, got {pdts}")
            self.upd_dtype = next(iter(pdts))
            for p in params:
                self._check_tensor(p.data, "parameter")
        self.apply_groups = list(apply_groups) if self.fused else None
        counts = []
        for g in grads:
            h, w = g.shape
            counts.append(((h + self.tile_h - 1) // self.tile_h) * ((w + self.tile_w - 1) // self.tile_w))
        self.tile_counts = counts
        self.tile0 = [sum(counts[:i]) for i in range(len(counts))]
        self.n_tiles = sum(counts)
        self.ppt = nat.gather_partials_per_tile(self.tile_h, self.tile_w, self.mp, self.np)
        # NS tile buffers, allocated on first use: a group whose step runs in
        # LDS (lds_step) never needs them.
        self._bufs = None
        self.updates = [] if self.fused else [torch.empty(g.shape, device=device, dtype=self.upd_dtype) for g in grads]
        self.upd_scales = list(upd_scales)
        self._sig = None
        self._bound = None
        self.desc = None
        self.bind(grads, moms, mus, nesterovs)

    # -- NS tile buffers ------------------------------------------------------
    def _buffers(self):
        if self._bufs is None:
            shape = (self.n_tiles, self.mp, self.np)
            # X ping-pongs between tiles and alt through the NS iterations.
            self._bufs = (
                torch.empty(shape, device=self.device, dtype=torch.bfloat16),
                torch.empty(shape, device=self.device, dtype=torch.bfloat16),
                torch.empty((self.n_tiles, self.ppt), device=self.device, dtype=torch.float32),
                torch.empty((self.n_tiles,), device=self.device, dtype=torch.float32),
            )
        return self._bufs

    @property
    def tiles(self) -> torch.Tensor:
        return self._buffers()[0]

    @property
    def alt(self) -> torch.Tensor:
        return self._buffers()[1]

    @property
    def partials(self) -> torch.Tensor:
        return self._buffers()[2]

    @property
    def inv(self) -> torch.Tensor:
        return self._buffers()[3]

    # -- descriptors -----------------------------------------------------
    @staticmethod
    def _check_tensor(t: torch.Tensor, what: str) -> None:
        if t.ndim != 2:
            raise ValueError(f"{what} must be 2-D, got shape {tuple(t.shape)}")
        if t.stride(1) != 1 and t.shape[1] > 1:
            raise ValueError(f"{what} must be row-major (stride(1) == 1), got strides {t.stride()}")

    def bind(self, grads, moms, mus, nesterovs) -> bool:
        """Rewrite the device descriptor table if any pointer or momentum
        setting changed (in place: the table keeps its device address, so a
        captured graph that reads it sees the new pointers). Returns True if
        the table was written. The table holds raw pointers, so the group keeps
        the bound grads and momentum buffers alive until release()."""
        sig = tuple(
            (g.data_ptr(), None if m is None else m.data_ptr(), float(mu), bool(nv))
            for g, m, mu, nv in zip(grads, moms, mus, nesterovs)
        )
        if sig == self._sig:
            return False
        descs = []
        for i, (g, m) in enumerate(zip(grads, moms)):
            self._check_tensor(g, "grad")
            if g.dtype != self.dtype:
                raise TypeError(f"bucket dtype {self.dtype} but grad dtype {g.dtype}")
            if m is not None:
                self._check_tensor(m, "momentum buffer")
            u = self.params[i].data if self.fused else self.updates[i]
            h, w = g.shape
            d = nat.ParamDesc()
            d.grad = g.data_ptr()
            d.momentum = m.data_ptr() if m is not None else None
            d.update = u.data_ptr()
            d.h, d.w = h, w
            d.ld_grad = g.stride(0) if h > 1 else w
            d.ld_mom = (m.stride(0) if h > 1 else w) if m is not None else 0
            d.ld_upd = u.stride(0) if h > 1 else w
            d.tile0 = self.tile0[i]
            d.R = (h + self.tile_h - 1) // self.tile_h
            d.C = (w + self.tile_w - 1) // self.tile_w
            d.upd_scale = self.upd_scales[i]
            d.mu = float(mus[i])
            d.nesterov = 1 if nesterovs[i] else 0
            d.group = self.apply_groups[i] if self.fused else 0
            descs.append(d)
        table = nat.make_desc_table(descs, self.device)
        if self.desc is not None and self.desc.numel() == table.numel():
            self.desc.copy_(table)
        else:
            self.desc = table
        self._sig = sig
        self._bound = (list(grads), list(moms))
        return True

    def release(self) -> None:
        """Drop the references bind() took, once every launch that reads the
        bound tensors is enqueued and their owner keeps them (the optimizer's
        parameters hold their grads, its state the momentum buffers). Memory
        torch frees afterwards is reused only in stream order, after those
        launches. Without this, an eager loop with zero_grad(set_to_none=True)
        would keep the previous step's grads alive while backward allocates
        the next ones."""
        self._bound = None

    # -- launches ----------------------------------------------------------
    def gather(self) -> None:
        nat.momentum_gather(
            self.desc, len(self.tile0), self.n_tiles, self.tile_h, self.tile_w, self.mp, self.np,
            self.dtype, self.tiles, self.partials,
        )
        nat.tile_scale(self.partials, self.ppt, self.n_tiles, self.inv)

    @staticmethod
    def _rng(t, start, count):
        return None if t is None else t[start : start + count]

    def ns(self, start: int, count: int, steps: int, workspace: torch.Tensor, sub_batch: int) -> None:
        if count <= 0:
            return
        r = self._rng
        nat.ns5(
            r(self.tiles, start, count), r(self.alt, start, count),
            self.inv[start : start + count], count, self.mp, self.np, steps,
            workspace, sub_batch, family=self.ns_family, round_once=self.round_once, rows=self.m,
        )

    def ns_untile_ok(self, steps: int) -> bool:
        """True when the untile with WD/LR can run inside the last NS
        iteration (himuon_ns5_untile_apply): fused mode, 512 x 512 NS tiles
        without transpose, family "auto", steps >= 2, fp32 or bf16 parameters."""
        return self.fused and nat.ns5_untile_apply_supported(
            self.mp, self.np, self.tile_h, self.tile_w, steps, self.upd_dtype, self.ns_family, self.round_once)

    def ns_untile(self, start: int, count: int, steps: int, workspace: torch.Tensor, sub_batch: int,
                  scale_alpha: torch.Tensor) -> None:
        """NS of tiles start .. start + count - 1 with the untile and the WD/LR
        of scale_alpha fused into the last iteration (the parameters of those
        tiles are updated; untile() must not run for them afterwards)."""
        if count <= 0:
            return
        r = self._rng
        nat.ns5_untile_apply(
            r(self.tiles, start, count), r(self.alt, start, count), self.inv[start : start + count], count,
            self.mp, self.np, steps, workspace, sub_batch, self.desc, len(self.tile0), start, self.tile_h,
            self.tile_w, self.upd_dtype, scale_alpha, family=self.ns_family, round_once=self.round_once,
            rows=self.m,
        )

    def lds_step_ok(self) -> bool:
        """True when the whole step of this group runs as one launch per chunk
        (himuon_lds_step): fused mode, 128 x 128 NS tiles without transpose,
        fp32/bf16 grads and parameters."""
        return (self.fused and self.ns_family != "block128"
                and nat.lds_step_supported(self.tile_h, self.tile_w, self.dtype, self.upd_dtype))

    def lds_step(self, start: int, count: int, steps: int, scale_alpha: torch.Tensor) -> None:
        """Momentum, gather, normaliser, NS and the untile with the WD/LR of
        scale_alpha for tiles start .. start + count - 1, one launch; the tile
        buffers are not used."""
        if count <= 0:
            return
        nat.lds_step(self.desc, len(self.tile0), start, count, self.tile_h, self.tile_w, self.dtype,
                     self.upd_dtype, steps, scale_alpha, round_once=self.round_once)

    def result(self, steps: int) -> torch.Tensor:
        """Buffer holding the NS output after `steps` iterations."""
        return self.tiles if steps % 2 == 0 else self.alt

    def untile(self, steps: int = 5, scale_alpha: torch.Tensor | None = None) -> None:
        """Write the update tensors, or, in fused mode, apply the WD/LR of
        scale_alpha (device (s_g, alpha_g) per group) to the parameters."""
        if self.fused:
            if scale_alpha is None:
                raise ValueError("fused TileGroup.untile needs the (scale, alpha) device table")
            nat.untile_apply(
                self.desc, len(self.tile0), self.n_tiles, self.tile_h, self.tile_w, self.mp, self.np,
                self.upd_dtype, self.result(steps), scale_alpha,
            )
            return
        nat.untile(
            self.desc, len(self.tile0), self.n_tiles, self.tile_h, self.tile_w, self.mp, self.np,
            self.upd_dtype, self.result(steps),
        )

    def workspace_bytes(self, sub_batch: int) -> int:
        return nat.ns5_workspace_bytes(sub_batch, self.mp, self.np)

    def default_sub_batch(self) -> int:
        return nat.default_sub_batch(self.n_tiles, self.mp, self.np)


class ApplyTables:
    """Device descriptor tables for the WD + LR application of a list of
    (param, update, group_idx), one table per (param dtype, update dtype)
    pair, built once (pointers must stay put: the graph path's updates and
    the parameters do). Entries the kernel cannot take (non-contiguous,
    misaligned, other dtypes, more than APPLY_MAX_GROUPS groups) are left to
    the torch ops of the reference (``fallback``)."""

    def __init__(self, entries):
        chunk = int(nat.load().himuon_apply_chunk_elems())
        by_pair: dict[tuple, list] = {}
        self.fallback = []
        for p, u, gi in entries:
            pd, ud = p.data, u
            ok = (
                pd.is_cuda and ud.is_cuda and pd.is_contiguous() and ud.is_contiguous()
                and pd.numel() == ud.numel() and pd.dtype in nat.DTYPE_CODES and ud.dtype in nat.DTYPE_CODES
                and pd.data_ptr() % 16 == 0 and ud.data_ptr() % 16 == 0 and gi < nat.APPLY_MAX_GROUPS
            )
            if ok:
                by_pair.setdefault((pd.dtype, ud.dtype), []).append((pd, ud, gi))
            else:
                self.fallback.append((p, u, gi))
        self.launches = []  # (table, n_descs, n_chunks, pdtype, udtype)
        for (pdt, udt), lst in by_pair.items():
            descs, c0 = [], 0
            for pd, ud, gi in lst:
                d = nat.ApplyDesc()
                d.param, d.update, d.numel, d.chunk0, d.group = pd.data_ptr(), ud.data_ptr(), pd.numel(), c0, gi
                descs.append(d)
                c0 += -(-pd.numel() // chunk)
            self.launches.append((nat.apply_desc_table(descs, lst[0][0].device), len(descs), c0, pdt, udt))

    def run(self, scales: list[float], alphas: list[float]) -> None:
        for table, n, n_chunks, pdt, udt in self.launches:
            nat.apply_updates(table, n, n_chunks, pdt, udt, scales, alphas)


class AdamwTables:
    """Device descriptor tables for the AdamW fallback step of a list of
    (grad, moment1, moment2, update, step, group_idx), one table (and one
    launch pair) per grad dtype, built once: every pointer must stay put, as
    the graph path requires of grads anyway. Entries the kernel cannot take
    (non-contiguous, misaligned, mixed or other dtypes, more than
    ADAMW_MAX_GROUPS groups) are returned in ``fallback`` for the reference's
    torch ops."""

    def __init__(self, entries):
        chunk = nat.adamw_chunk_elems()
        by_dtype: dict[torch.dtype, list] = {}
        self.fallback = []
        for e in entries:
            g, m, v, u, st, gi = e
            ts = (g, m, v, u)
            ok = (
                all(t.is_cuda and t.is_contiguous() and t.data_ptr() % 16 == 0 and t.dtype == g.dtype
                    and t.numel() == g.numel() for t in ts)
                and g.dtype in nat.DTYPE_CODES and st.is_cuda and st.dtype == torch.float32 and st.numel() == 1
                and g.numel() > 0 and gi < nat.ADAMW_MAX_GROUPS
            )
            if ok:
                by_dtype.setdefault(g.dtype, []).append(e)
            else:
                self.fallback.append(e)
        self.launches = []  # (table, n_descs, n_chunks, dtype, bias scratch)
        for dt, lst in by_dtype.items():
            descs, c0 = [], 0
            for g, m, v, u, st, gi in lst:
                d = nat.AdamwDesc()
                d.grad, d.moment1, d.moment2, d.update = g.data_ptr(), m.data_ptr(), v.data_ptr(), u.data_ptr()
                d.step, d.numel, d.chunk0, d.group = st.data_ptr(), g.numel(), c0, gi
                descs.append(d)
                c0 += -(-g.numel() // chunk)
            dev = lst[0][0].device
            bias = torch.zeros(2 * len(descs), device=dev, dtype=torch.float32)
            self.launches.append((nat.adamw_desc_table(descs, dev), len(descs), c0, dt, bias))

    def run(self, beta1s: list[float], beta2s: list[float], epss: list[float]) -> None:
        for table, n, n_chunks, dt, bias in self.launches:
            nat.adamw_step(table, n, n_chunks, dt, beta1s, beta2s, epss, bias)


class _NsPlan:
    """Device state of ``newton_schulz`` for one (batch shape, dtype, device,
    rounding form, kernel family): a tile group over its own input and output
    buffers, the sub-batch and the NS workspace, built once, and per step
    count a hipGraph of its launches (gather, normaliser, NS, untile),
    captured on first use. A call copies the input into ``xin``, replays the
    graph and copies the result out of ``out``: it neither allocates device
    state (beyond the returned tensor) nor rewrites the descriptor table, and
    costs one replay instead of a dozen or more host launches."""

    def __init__(self, n: int, M: int, N: int, dtype: torch.dtype, device, round_once: bool, family: str):
        self.xin = torch.empty((n * M, N), device=device, dtype=dtype)
        self.grp = TileGroup(
            params=[self.xin], grads=[self.xin], moms=[None], tile_h=M, tile_w=N, upd_scales=[1.0],
            mus=[0.0], nesterovs=[False], device=device, dtype=dtype, round_once=round_once, ns_family=family,
        )
        self.out = self.grp.updates[0]
        self.sub_batch = self.grp.default_sub_batch()
        self.ws = torch.empty(max(1, self.grp.workspace_bytes(self.sub_batch)), device=device, dtype=torch.uint8)
        self.grp.tiles  # allocate the tile buffers now, not inside a capture
        self.graphs: "dict[int, torch.cuda.CUDAGraph]" = {}
        # recorded into a caller's graph: that graph holds these buffers'
        # addresses, so the plan is never dropped
        self.pinned = False

    def _launches(self, steps: int) -> None:
        g = self.grp
        g.gather()
        g.ns(0, g.n_tiles, steps, self.ws, self.sub_batch)
        g.untile(steps)

    def run(self, steps: int) -> torch.Tensor:
        if torch.cuda.is_current_stream_capturing():
            # inside the caller's capture: record the launches there
            self.pinned = True
            self._launches(steps)
            return self.out
        graph = self.graphs.get(steps)
        if graph is None:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._launches(steps)
            self.graphs[steps] = graph
        graph.replay()
        return self.out


_NS_PLANS: "dict[tuple, _NsPlan]" = {}
_NS_PLANS_MAX = 8


def newton_schulz(G: torch.Tensor, steps: int = 5, family: str = "auto") -> torch.Tensor:
    """Batched NS5 of ``G`` (..., M, N) on the HIP path; same shape and dtype.

    The batch is viewed as one (B*M, N) matrix cut into M x N tiles, so the
    gather/untile kernels handle the cast, the transpose-if-tall and the
    padding (himuon.py:263-284, test_kernels.py:176-198). A 2-D ``G`` takes
    the reference's 2-D rounding of the third product (torch.addmm,
    himuon.py:249-253); a batched one that of fused_bmm_add. The device state
    for a shape is built on its first call and reused (at most _NS_PLANS_MAX
    shapes are kept, the least recently used dropped first, except those
    recorded into a caller's graph); the result is a new tensor.
    ``family``: the NS kernel family (comparison runs; "auto" otherwise)."""
    assert G.ndim >= 2
    if not G.is_cuda:
        raise RuntimeError("HiMuon.newton_schulz runs on the HIP device only (no CPU path)")
    M, N = G.shape[-2], G.shape[-1]
    dtype = G.dtype if G.dtype in nat.DTYPE_CODES else torch.float32
    n = G.numel() // (M * N) if M * N else 0
    if n == 0:
        return torch.empty_like(G)
    key = (n, M, N, dtype, G.device, G.ndim == 2, family)
    plan = _NS_PLANS.pop(key, None)
    if plan is None:
        if len(_NS_PLANS) >= _NS_PLANS_MAX:
            old = next((k for k, v in _NS_PLANS.items() if not v.pinned), None)
            if old is not None:
                _NS_PLANS.pop(old)
        plan = _NsPlan(n, M, N, dtype, G.device, G.ndim == 2, family)
    _NS_PLANS[key] = plan  # most recently used last
    plan.xin.view(G.shape).copy_(G)
    return plan.run(steps).view(G.shape).to(G.dtype, copy=True)
