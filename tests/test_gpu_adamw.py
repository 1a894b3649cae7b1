"""GPU parity of the fused AdamW fallback step (himuon_adamw_step) against the
reference's torch ops (himuon.py:359-372, `_compute_adamw_step`):

    step.add_(1); m.lerp_(g, 1 - b1); v.lerp_(g.square(), 1 - b2)
    update = (m / (1 - b1**step)) / (v.sqrt() / (1 - b2**step)**0.5 + eps)

bit for bit on the GPU for fp32/bf16/fp16 moments, ragged sizes and several
param groups (including lerp weights >= 0.5, the other branch of torch's
lerp), over more steps than the first one where the device powf leaves
correct rounding; the kernel's bias corrections equal torch's; moments and
update equal the CPU oracle given those bias corrections; and at the
optimizer level (eager and hipGraph replay) the parameters of AdamW groups
equal a restatement of the reference's step bit for bit.
"""

from __future__ import annotations


import numpy as np
import pytest
import torch

from oracle import himuon_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from himuon_amd.engine import AdamwTables
    from himuon_amd.optimizers.himuon import HiMuon

DEV = "cuda"
NAMES = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}
# (beta1, beta2, eps) per group; the last has lerp weights 0.7 / 0.55 (>= 0.5)
GROUPS = [(0.95, 0.95, 1e-8), (0.9, 0.999, 1e-6), (0.3, 0.45, 1e-8)]
# ragged: a single element, below one vector, not a multiple of 8, several
# 4096-element chunks with a tail, and a larger one
SHAPES = [(1,), (5,), (3, 7), (4096 * 3 + 5,), (257, 129), (1024, 700)]


def _ref_adamw(g, st, betas, eps):
    """The reference's op chain on the GPU (himuon.py:366-372)."""
    step = st["step"]
    step.add_(1)
    m, v = st["moment1"], st["moment2"]
    m.lerp_(g, 1 - betas[0])
    v.lerp_(g.square(), 1 - betas[1])
    bc1 = 1 - betas[0] ** step
    bc2 = 1 - betas[1] ** step
    return (m / bc1) / (v.sqrt() / bc2**0.5 + eps)


def _bits(t):
    t = t.detach().cpu()
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16).numpy()


def _make(dtype, seed=3):
    gen = torch.Generator().manual_seed(seed)
    params = []
    for k, shp in enumerate(SHAPES):
        gi = k % len(GROUPS)
        g = torch.empty(shp, dtype=dtype, device=DEV)
        st = {"step": torch.zeros((), device=DEV), "moment1": torch.zeros_like(g), "moment2": torch.zeros_like(g)}
        ref = {k2: v.clone() for k2, v in st.items()}
        params.append({"g": g, "st": st, "ref": ref, "u": torch.empty_like(g), "gi": gi})
    return params, gen


def _hyper():
    return [b[0] for b in GROUPS], [b[1] for b in GROUPS], [b[2] for b in GROUPS]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_adamw_kernel_bit_exact_vs_torch_ops(dtype):
    params, gen = _make(dtype)
    tables = AdamwTables(
        [(q["g"], q["st"]["moment1"], q["st"]["moment2"], q["u"], q["st"]["step"], q["gi"]) for q in params]
    )
    assert not tables.fallback and len(tables.launches) == 1
    b1s, b2s, eps = _hyper()
    for step in range(7):  # beta 0.95: step 6 is the first where powf is not correctly rounded
        for q in params:
            q["g"].copy_((torch.randn(q["g"].shape, generator=gen) * 1e-3).to(dtype).to(DEV))
        tables.run(b1s, b2s, eps)
        for q in params:
            b1, b2, e = GROUPS[q["gi"]]
            u_ref = _ref_adamw(q["g"], q["ref"], (b1, b2), e)
            assert q["st"]["step"].item() == q["ref"]["step"].item() == step + 1
            for name in ("moment1", "moment2"):
                assert np.array_equal(_bits(q["st"][name]), _bits(q["ref"][name])), (step, name, q["g"].shape)
            assert u_ref.dtype == dtype
            assert np.array_equal(_bits(q["u"]), _bits(u_ref)), (step, "update", q["g"].shape)


def test_adamw_bias_corrections_match_torch():
    """The prep kernel's (1 - b1**step, (1 - b2**step)**0.5) equal torch's
    fp32 ops on the GPU at every step 1..40 (the device powf, not a correctly
    rounded power: the oracle's adamw_bias differs at some of these steps)."""
    g = torch.zeros(16, device=DEV)
    st = torch.zeros((), device=DEV)
    m, v, u = torch.zeros_like(g), torch.zeros_like(g), torch.empty_like(g)
    for betas in ((0.95, 0.95), (0.9, 0.999)):
        st.zero_()
        tables = AdamwTables([(g, m, v, u, st, 0)])
        bias = tables.launches[0][4]
        differs = 0
        for s in range(1, 41):
            tables.run([betas[0]], [betas[1]], [1e-8])
            ts = torch.tensor(float(s), device=DEV)
            bc1 = 1 - betas[0] ** ts
            sbc2 = (1 - betas[1] ** ts) ** 0.5
            got = bias.cpu()
            assert got[0].item() == bc1.item() and got[1].item() == sbc2.item(), (betas, s)
            differs += int(np.float32(got[0].item()) != O.adamw_bias(betas[0], s))
        assert st.item() == 40.0
        if betas[0] == 0.95:
            assert differs > 0  # the device powf is not correctly rounded (steps 6, 12, 13, ...)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_adamw_kernel_matches_oracle_given_bias(dtype):
    params, gen = _make(dtype, seed=4)
    tables = AdamwTables(
        [(q["g"], q["st"]["moment1"], q["st"]["moment2"], q["u"], q["st"]["step"], q["gi"]) for q in params]
    )
    bias = tables.launches[0][4]
    b1s, b2s, eps = _hyper()
    om = [np.zeros(q["g"].numel(), np.float32) for q in params]
    ov = [np.zeros(q["g"].numel(), np.float32) for q in params]
    # fp16 at 1e-3 would underflow v (and eps) to zero: use a scale it can hold
    scale = 1e-1 if dtype == torch.float16 else 1e-3
    for step in range(4):
        for q in params:
            q["g"].copy_((torch.randn(q["g"].shape, generator=gen) * scale).to(dtype).to(DEV))
        tables.run(b1s, b2s, eps)
        bb = bias.cpu().numpy()
        for i, q in enumerate(params):
            b1, b2, e = GROUPS[q["gi"]]
            u, om[i], ov[i], s, _ = O.adamw_step(
                q["g"].float().cpu().numpy().ravel(), om[i], ov[i], step, (b1, b2), e, NAMES[dtype],
                bias=(bb[2 * i], bb[2 * i + 1]),
            )
            assert s == step + 1
            assert np.array_equal(q["st"]["moment1"].float().cpu().numpy().ravel(), om[i])
            assert np.array_equal(q["st"]["moment2"].float().cpu().numpy().ravel(), ov[i])
            assert np.array_equal(q["u"].float().cpu().numpy().ravel(), u, equal_nan=True)


def _model(dtype, seed=0):
    torch.manual_seed(seed)
    emb = torch.nn.Parameter((torch.randn(1000, 64) * 0.02).to(dtype).to(DEV))   # embedding-like, AdamW
    w = torch.nn.Parameter((torch.randn(256, 512) * 0.02).to(dtype).to(DEV))    # Muon
    norm = torch.nn.Parameter(torch.ones(64, dtype=dtype, device=DEV))           # 1-D, AdamW
    bias = torch.nn.Parameter(torch.zeros(257, dtype=dtype, device=DEV))         # ragged 1-D, AdamW
    return [emb, w, norm, bias]


def _groups(ps):
    emb, w, norm, bias = ps
    return [
        {"params": [w], "use_muon": True, "weight_decay": 0.1},
        {"params": [emb], "use_muon": False, "lr": 2e-3, "weight_decay": 0.1},
        {"params": [norm, bias], "use_muon": False, "lr": 1e-3, "weight_decay": 0.0,
         "adamw_betas": (0.9, 0.999), "adamw_eps": 1e-6},
    ]


def _seed(ps, seed):
    gen = torch.Generator().manual_seed(seed)
    for p in ps:
        vals = (torch.randn(p.shape, generator=gen) * 1e-3).to(p.dtype).to(DEV)
        if p.grad is None:
            p.grad = torch.empty_like(p)
        p.grad.copy_(vals)


def _reference_adamw_params(ps, groups, n_steps, seed0):
    """The reference's AdamW-group step on copies: torch op chain, then
    p.mul_(1 - lr*wd) (wd > 0) and p.add_(update, alpha=-lr)."""
    state = {}
    for k in range(n_steps):
        _seed(ps, seed0 + k)
        for gr in groups[1:]:
            b1, b2 = gr.get("adamw_betas", (0.95, 0.95))
            eps = gr.get("adamw_eps", 1e-8)
            for p in gr["params"]:
                st = state.setdefault(id(p), {"step": torch.zeros((), device=DEV),
                                              "moment1": torch.zeros_like(p.grad),
                                              "moment2": torch.zeros_like(p.grad)})
                u = _ref_adamw(p.grad, st, (b1, b2), eps)
                if gr["weight_decay"] > 0:
                    p.data.mul_(1 - gr["lr"] * gr["weight_decay"])
                p.data.add_(u, alpha=-gr["lr"])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cuda_graph", [False, True])
def test_optimizer_adamw_groups_match_reference(dtype, cuda_graph):
    ps = _model(dtype)
    ref = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    opt = HiMuon(_groups(ps), lr=0.02, tile_size=256, cuda_graph=cuda_graph, cuda_graph_warmup=2)
    n = 6
    for k in range(n):
        _seed(ps, 100 + k)
        opt.step()
    if cuda_graph:
        assert opt._cuda_graph is not None
    _reference_adamw_params(ref, _groups(ref), n, 100)
    for i in (0, 2, 3):  # the AdamW-group parameters
        assert np.array_equal(_bits(ps[i].data), _bits(ref[i].data)), i
        st = opt.state[ps[i]]
        assert st["step"].item() == n


def test_optimizer_adamw_non_contiguous_grad_falls_back():
    """A grad the kernel cannot take (non-contiguous) runs the reference's
    torch ops, with the same result."""
    ps = _model(torch.float32, seed=1)
    ref = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    opt = HiMuon(_groups(ps), lr=0.02, tile_size=256, cuda_graph=False)
    for k in range(3):
        _seed(ps, 300 + k)
        ps[0].grad = ps[0].grad.t().contiguous().t()  # same values, transposed strides
        assert not ps[0].grad.is_contiguous()
        opt.step()
    assert opt._adamw_tables is not None and len(opt._adamw_tables.fallback) == 1
    _reference_adamw_params(ref, _groups(ref), 3, 300)
    for i in (0, 2, 3):
        assert np.array_equal(_bits(ps[i].data), _bits(ref[i].data)), i
