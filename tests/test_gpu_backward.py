"""Straight-through backward parity: HIP scatter-add vs the oracle's autograd."""

from __future__ import annotations

import pytest
import torch

import jointkv_amd as jkv
from oracle import jointkv_oracle as ref

pytestmark = pytest.mark.gpu

GRAD_RTOL = 1e-5  # relative (per table, Frobenius) tolerance on fp32 codebook grads


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.cpu().double() - b.cpu().double()).norm() / b.cpu().double().norm().clamp_min(1e-30))


def test_known_answer_one_dimensional(device):
    # tests/test_closed_loop_vq.py:131-162 of the reference
    states = torch.tensor([[[[0.1]]]], device=device, requires_grad=True)
    tables = torch.tensor([[[[0.0], [1.0], [10.0], [20.0]]]], device=device, requires_grad=True)
    out, codes = jkv.hard_residual_vq_exits(states, tables, prefixes=(1,), straight_through_states=False)
    out[1].sum().backward()
    assert int(codes.item()) == 0
    assert tables.grad[0, 0, 0].item() == 1.0
    assert tables.grad[0, 0, 1:].count_nonzero() == 0
    assert states.grad is None


@pytest.mark.parametrize("deterministic", [False, True])
def test_grouped_residual_backward_matches_oracle(device, deterministic):
    # config 5 geometry per layer (reduced T): V states fp16, G2 fp32 masters,
    # upstream dL/dV̂ ~ N(0, 1e-3) stored fp16
    gen = torch.Generator().manual_seed(8607)
    states = ref.synthetic_states(gen, 4, 8, 256)
    tables = ref.synthetic_tables(gen, (8, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2)
    upstream = (torch.randn(4, 8, 256, 128, generator=gen) * 1e-3 ** 0.5).half()
    x = states.to(device).requires_grad_()
    t = tables.to(device).requires_grad_()
    exits, codes = jkv.hard_grouped_residual_vq(x, t, prefixes=(2,), deterministic_backward=deterministic)
    exits[2].backward(upstream.to(device))
    expect = ref.table_gradient([upstream], [2], codes.cpu(), (128, 2, 256, 8)).reshape(tables.shape)
    assert _rel(t.grad, expect) <= GRAD_RTOL
    assert torch.equal(x.grad.cpu(), upstream)
    if deterministic:
        t2 = tables.to(device).requires_grad_()
        e2, _c = jkv.hard_grouped_residual_vq(states.to(device), t2, prefixes=(2,), deterministic_backward=True)
        e2[2].backward(upstream.to(device))
        assert torch.equal(t.grad, t2.grad), "deterministic backward is not bit-reproducible"


def test_multiple_exits_and_fp32_states(device):
    gen = torch.Generator().manual_seed(43)
    states = torch.randn(2, 2, 40, 8, generator=gen)
    tables = torch.randn(2, 3, 16, 8, generator=gen)
    x = states.to(device).requires_grad_()
    t = tables.to(device).requires_grad_()
    exits, codes = jkv.hard_residual_vq_exits(x, t, prefixes=(2, 3))
    g2 = torch.randn(exits[2].shape, generator=gen)
    g3 = torch.randn(exits[3].shape, generator=gen)
    (exits[2] * g2.to(device) + exits[3] * g3.to(device)).sum().backward()
    # oracle autograd on the same inputs
    xs = states.clone().requires_grad_()
    ts = tables.clone().requires_grad_()
    r_exits, r_codes = ref.hard_residual_vq_exits(xs, ts, prefixes=(2, 3))
    assert torch.equal(codes.cpu(), r_codes)
    (r_exits[2] * g2 + r_exits[3] * g3).sum().backward()
    assert _rel(t.grad, ts.grad) <= GRAD_RTOL
    torch.testing.assert_close(x.grad.cpu(), xs.grad, rtol=0, atol=0)


def test_grouped_cq_backward_and_frozen_key_tables(device):
    gen = torch.Generator().manual_seed(21)
    states = ref.synthetic_states(gen, 1, 8, 128)
    books = ref.synthetic_tables(gen, (8, 32, 256, 4), (1.0,), stage_axis=0)
    upstream = torch.randn(1, 8, 128, 128, generator=gen).half()
    b = books.to(device).requires_grad_()
    out, codes = jkv.hard_grouped_cq(states.to(device), b)
    out.backward(upstream.to(device))
    expect = ref.table_gradient([upstream], [1], codes.cpu()[..., None], (256, 1, 256, 4)).reshape(books.shape)
    assert _rel(b.grad, expect) <= GRAD_RTOL
    # frozen tables (requires_grad False) get no gradient, states still do
    frozen = books.to(device)
    x = states.to(device).requires_grad_()
    o2, _ = jkv.hard_grouped_cq(x, frozen)
    o2.float().sum().backward()
    assert frozen.grad is None and x.grad is not None


def test_gradient_sum_invariant_full_layer(device):
    # size-independent property at config-5 layer size: per stage the codebook
    # gradient sums to the summed upstream gradient of each group.
    gen = torch.Generator().manual_seed(8613)
    states = ref.synthetic_states(gen, 4, 8, 2048).to(device)
    tables = ref.synthetic_tables(gen, (8, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2).to(device).requires_grad_()
    upstream = (torch.randn(4, 8, 2048, 128, generator=gen) * 1e-3 ** 0.5).half().to(device)
    exits, codes = jkv.hard_grouped_residual_vq(states, tables, prefixes=(2,))
    exits[2].backward(upstream)
    per_group = upstream.double().reshape(4, 8, 2048, 16, 8).sum(dim=(0, 2))  # [8,16,8]
    for s in range(2):
        got = tables.grad[:, :, s].double().sum(dim=2)  # [8,16,8]
        torch.testing.assert_close(got, per_group, rtol=1e-4, atol=1e-4)
    # occupancy: every row lands in exactly one bin per stage
    counts = torch.zeros(8 * 16 * 2 * 256, device=device)
    flat = codes.long().permute(1, 3, 4, 0, 2).reshape(8 * 16, 2, -1)
    idx = (torch.arange(128, device=device)[:, None, None] * 2 + torch.arange(2, device=device)[None, :, None]) * 256 + flat
    counts.index_add_(0, idx.reshape(-1), torch.ones(idx.numel(), device=device))
    assert int(counts.sum()) == 4 * 2048 * 8 * 16 * 2


def _random_scatter_case(gen, batch, heads, tokens, groups, d, stages, n_exits, dtype, scale=0.03):
    codes = torch.randint(0, 256, (batch, heads, tokens, groups, stages), generator=gen, dtype=torch.int32)
    grads = [(torch.randn(batch, heads, tokens, groups * d, generator=gen) * scale).to(dtype) for _ in range(n_exits)]
    return codes.to(torch.uint8), grads


EXACT_CASES = [
    # (B, H, T, G, d, S, exits): one chunk, row chunks (one head), several
    # exits, full-vector RVQ (d = 128 in 8-dim slices), grouped CQ (d = 4)
    (4, 8, 200, 16, 8, 2, (2,)),
    (4, 8, 2048, 16, 8, 2, (2,)),  # config-5 layer: 8192 rows per (head, group, stage) block
    (2, 8, 100, 16, 8, 2, (1, 2)),  # one block per (head, group, stage), two exits
    (4, 1, 2048, 16, 8, 2, (2,)),
    (4, 1, 2048, 16, 8, 2, (1, 2)),
    (2, 2, 300, 1, 128, 3, (1, 3)),
    (2, 2, 100, 32, 4, 1, (1,)),
]


@pytest.mark.parametrize("case", EXACT_CASES)
def test_fp16_scatter_is_the_correctly_rounded_exact_sum(device, case):
    # fp16 gradients are summed in exact fixed point: every bin equals the fp32
    # rounding of the exact sum (fp64 is exact at these sizes), bit for bit.
    from jointkv_amd import _ops

    batch, heads, tokens, groups, d, stages, exits = case
    gen = torch.Generator().manual_seed(8621 + tokens + d + len(exits))
    codes, grads = _random_scatter_case(gen, batch, heads, tokens, groups, d, stages, len(exits), torch.float16)
    shape = (heads * groups, stages, 256, d)
    expect = ref.table_gradient(grads, exits, codes, shape, accumulate=torch.float64).float()
    got = torch.zeros(shape, device=device)
    _ops.rvq_scatter_grad([g.to(device) for g in grads], exits, codes.to(device), got, group_dim=d)
    assert torch.equal(got.cpu(), expect)
    # accumulation into an existing gradient: one more fp32 add per bin
    _ops.rvq_scatter_grad([g.to(device) for g in grads], exits, codes.to(device), got, group_dim=d)
    assert torch.equal(got.cpu(), expect + expect)


def test_scatter_global_atomic_path(device):
    # d not a multiple of 4 takes global fp32 atomics
    from jointkv_amd import _ops

    gen = torch.Generator().manual_seed(8623)
    codes, grads = _random_scatter_case(gen, 2, 2, 150, 3, 6, 2, 2, torch.float16)
    shape = (6, 2, 256, 6)
    expect = ref.table_gradient(grads, (1, 2), codes, shape)
    got = torch.zeros(shape, device=device)
    _ops.rvq_scatter_grad([g.to(device) for g in grads], (1, 2), codes.to(device), got, group_dim=6)
    assert _rel(got, expect) <= GRAD_RTOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("deterministic", [False, True])
def test_bf16_fp32_scatter_matches_oracle(device, dtype, deterministic):
    from jointkv_amd import _ops

    gen = torch.Generator().manual_seed(8629)
    codes, grads = _random_scatter_case(gen, 2, 4, 600, 32, 4, 1, 1, dtype)
    expect = ref.table_gradient(grads, (1,), codes, (128, 1, 256, 4))
    got = torch.zeros(128, 1, 256, 4, device=device)
    _ops.rvq_scatter_grad([g.to(device) for g in grads], (1,), codes.to(device), got, group_dim=4,
                          deterministic=deterministic)
    assert _rel(got, expect) <= GRAD_RTOL
    if deterministic:
        again = torch.zeros_like(got)
        _ops.rvq_scatter_grad([g.to(device) for g in grads], (1,), codes.to(device), again, group_dim=4,
                              deterministic=True)
        assert torch.equal(got, again)


@pytest.mark.parametrize("heads", [2, 8])
def test_fp16_scatter_nonfinite_gradients(device, heads):
    # inf / nan slices: the IEEE outcome of a floating-point sum per bin
    # (2 heads: one block per (head, group) with row chunks; 8 heads: one
    # block per (head, group, stage))
    from jointkv_amd import _ops

    gen = torch.Generator().manual_seed(8641)
    codes, grads = _random_scatter_case(gen, 1, heads, 3000, 16, 8, 2, 1, torch.float16)
    g = grads[0]
    g[0, 0, 5, 3] = float("inf")
    g[0, 1, 2999, 17] = float("-inf")
    g[0, 1, 100, 40] = float("nan")
    expect = ref.table_gradient([g], (2,), codes, (heads * 16, 2, 256, 8), accumulate=torch.float64).float()
    got = torch.zeros(heads * 16, 2, 256, 8, device=device)
    _ops.rvq_scatter_grad([g.to(device)], (2,), codes.to(device), got, group_dim=8)
    got = got.cpu()
    assert torch.equal(torch.isnan(got), torch.isnan(expect))
    assert torch.equal(torch.isinf(got), torch.isinf(expect))
    assert torch.equal(got[torch.isinf(got)], expect[torch.isinf(expect)])
    finite = torch.isfinite(expect)
    torch.testing.assert_close(got[finite], expect[finite], rtol=1e-5, atol=1e-6)


def test_scatter_misaligned_gradient_view(device):
    # a contiguous view whose start is not aligned to d elements
    from jointkv_amd import _ops

    gen = torch.Generator().manual_seed(8647)
    codes, grads = _random_scatter_case(gen, 1, 2, 300, 16, 8, 2, 1, torch.float16)
    flat = torch.zeros(grads[0].numel() + 1, dtype=torch.float16)
    flat[1:] = grads[0].reshape(-1)
    view = flat.to(device)[1:].view(grads[0].shape)
    assert view.data_ptr() % 16 != 0
    expect = ref.table_gradient(grads, (2,), codes, (32, 2, 256, 8), accumulate=torch.float64).float()
    for deterministic in (False, True):
        got = torch.zeros(32, 2, 256, 8, device=device)
        _ops.rvq_scatter_grad([view], (2,), codes.to(device), got, group_dim=8, deterministic=deterministic)
        assert torch.equal(got.cpu(), expect)


MANY_CASES = [
    # (jobs, B, H, T, G, d, S, exits, dtype)
    (5, 4, 8, 200, 16, 8, 2, (2,), torch.float16),     # one launch
    (70, 1, 2, 300, 16, 8, 2, (2,), torch.float16),    # 64 + 6 jobs: two launches
    (3, 2, 2, 100, 32, 4, 1, (1,), torch.float16),     # 4-dim slices
    (3, 2, 8, 100, 16, 8, 2, (1,), torch.float16),     # stage 2 reached by no exit: zeros stored
    (3, 2, 8, 100, 16, 8, 2, (1, 2), torch.float16),   # two exits: one scatter per job
    (3, 2, 4, 300, 32, 4, 1, (1,), torch.bfloat16),    # bf16: one scatter per job
]


@pytest.mark.parametrize("case", MANY_CASES)
def test_scatter_many_equals_per_job_scatters(device, case):
    # every job of the many-job call against its exact sum (fp16: the
    # correctly rounded fp64 sum, bit for bit) and against its own one-job
    # call; fresh tables hold the sums alone, given tables get them added
    from jointkv_amd import _ops

    jobs, batch, heads, tokens, groups, d, stages, exits, dtype = case
    print(f"scatter_many jobs={jobs} B={batch} H={heads} T={tokens} G={groups} d={d} S={stages} "
          f"exits={exits} {dtype}", flush=True)
    gen = torch.Generator().manual_seed(8700 + jobs + tokens + d)
    shape = (heads * groups, stages, 256, d)
    cases = [_random_scatter_case(gen, batch, heads, tokens, groups, d, stages, len(exits), dtype)
             for _ in range(jobs)]
    codes = [c.to(device) for c, _ in cases]
    grads = [[g.to(device) for g in gs] for _, gs in cases]
    fresh = _ops.rvq_scatter_grad_many(grads, exits, codes, group_dim=d, table_shape=shape)
    base = [torch.randn(shape, generator=gen) for _ in range(jobs)]
    added = _ops.rvq_scatter_grad_many(grads, exits, codes, [b.to(device) for b in base], group_dim=d)
    exact = dtype == torch.float16
    for j in range(jobs):
        c, gs = cases[j]
        if exact:
            expect = ref.table_gradient(gs, exits, c, shape, accumulate=torch.float64).float()
            assert torch.equal(fresh[j].cpu(), expect), f"job {j}"
            assert torch.equal(added[j].cpu(), base[j] + expect), f"job {j}"
            one = torch.zeros(shape, device=device)
            _ops.rvq_scatter_grad(grads[j], exits, codes[j], one, group_dim=d)
            assert torch.equal(one, fresh[j]), f"job {j}"
        else:
            expect = ref.table_gradient(gs, exits, c, shape)
            assert _rel(fresh[j], expect) <= GRAD_RTOL, f"job {j}"
            assert _rel(added[j].cpu() - base[j], expect) <= GRAD_RTOL, f"job {j}"


def test_scatter_many_overwrite_clears_tables_and_handles_nonfinite(device):
    # stored sums replace whatever the tables held (NaN here): codewords no
    # row picks come back 0, and a job with inf/nan slices gets the IEEE
    # outcome of a floating-point sum (its blocks clear their part first)
    from jointkv_amd import _ops

    gen = torch.Generator().manual_seed(8711)
    jobs, heads = 4, 8
    shape = (heads * 16, 2, 256, 8)
    cases = [_random_scatter_case(gen, 1, heads, 3000, 16, 8, 2, 1, torch.float16) for _ in range(jobs)]
    g = cases[2][1][0]
    g[0, 0, 5, 3] = float("inf")
    g[0, 1, 2999, 17] = float("-inf")
    g[0, 1, 100, 40] = float("nan")
    codes = [c.to(device) for c, _ in cases]
    # codewords 200..255 of stage 1 unused in job 0
    codes[0][..., 0] = codes[0][..., 0] % 200
    grads = [[x.to(device) for x in gs] for _, gs in cases]
    tables = [torch.full(shape, float("nan"), device=device) for _ in range(jobs)]
    out = _ops.rvq_scatter_grad_many(grads, (2,), codes, tables, group_dim=8, accumulate=False)
    for j in range(jobs):
        c, gs = cases[j]
        c = codes[j].cpu()
        expect = ref.table_gradient(gs, (2,), c, shape, accumulate=torch.float64).float()
        got = out[j].cpu()
        if j != 2:
            assert torch.equal(got, expect), f"job {j}"
            continue
        assert torch.equal(torch.isnan(got), torch.isnan(expect))
        assert torch.equal(torch.isinf(got), torch.isinf(expect))
        assert torch.equal(got[torch.isinf(got)], expect[torch.isinf(expect)])
        finite = torch.isfinite(expect)
        torch.testing.assert_close(got[finite], expect[finite], rtol=1e-5, atol=1e-6)
    assert bool((out[0].cpu()[:, 0, 200:] == 0).all())


def test_scatter_many_config5_equals_per_layer_scatters(device):
    # the V-only step's 32 value-table scatters at config 5's shape in one
    # launch, against each layer's own scatter (exact sums: bit for bit)
    from jointkv_amd import _ops

    print("scatter_many config 5 (32 x [4,8,2048,128])", flush=True)
    gen = torch.Generator(device=device).manual_seed(8607)
    codes = [torch.randint(0, 256, (4, 8, 2048, 16, 2), generator=gen, device=device, dtype=torch.int32)
             .to(torch.uint8) for _ in range(32)]
    grads = [[(torch.randn(4, 8, 2048, 128, generator=gen, device=device) * 1e-3 ** 0.5).half()] for _ in range(32)]
    fresh = _ops.rvq_scatter_grad_many(grads, (2,), codes, group_dim=8, table_shape=(128, 2, 256, 8))
    for layer in range(32):
        one = torch.zeros(128, 2, 256, 8, device=device)
        _ops.rvq_scatter_grad(grads[layer], (2,), codes[layer], one, group_dim=8)
        assert torch.equal(one, fresh[layer]), f"layer {layer}"
