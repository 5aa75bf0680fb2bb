"""Offline multi-exit additive coordinate refinement
(src/jointkv/nested_vq.py:178-215, 583-741): the CPU oracle pinned by
exhaustive search, the host function's argument checks, and the HIP nearest
search and refinement against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import jointkv_amd as jkv
from jointkv_amd import _ops
from oracle import additive_oracle as ora


def _problem(seed, batch, heads, tokens, dim, clusters, stages):
    gen = torch.Generator().manual_seed(seed)
    states = torch.randn(batch, heads, tokens, dim, generator=gen)
    tables = [torch.randn(heads, clusters, dim, generator=gen) * (0.7 ** s) for s in range(stages)]
    init = torch.randint(0, clusters, (batch, heads, tokens, stages), generator=gen)
    return states, tables, init


def _stage_objective(x, tabs, idx, stage, aff):
    """float64 weighted objective of every candidate k for `stage` over the
    exits in `aff`, the other stages at idx: [N, K]."""

    n, k = x.shape[0], tabs[stage].shape[0]
    out = np.zeros((n, k))
    for p, w in aff:
        base = np.zeros_like(x)
        for j in range(p):
            if j != stage:
                base += tabs[j][idx[:, j]]
        diff = (x - base)[:, None, :] - tabs[stage][None, :, :]
        out += w * np.square(diff).sum(-1)
    return out


@pytest.mark.parametrize("prefixes,weights", [((1, 2, 3), (1.0, 0.5, 2.0)), ((2, 3), (0.0, 1.0)), ((3,), (1.0,))])
def test_oracle_sweep_matches_exhaustive_search(prefixes, weights):
    states, tables, init = _problem(7, 1, 2, 40, 6, 12, 3)
    _out, idx, _hist, _init = ora.coordinate_refinement(states.numpy(), [t.numpy() for t in tables], init.numpy(),
                                                        prefixes, weights, sweeps=1)
    x_all = states.double().numpy()
    tabs_all = [t.double().numpy() for t in tables]
    checked = 0
    for h in range(2):
        x = x_all[0, h]
        final = idx[0, h]
        start = init.numpy()[0, h]
        for stage in range(2, -1, -1):
            aff = [(p, w) for p, w in zip(prefixes, weights) if p > stage and w > 0]
            if not aff:
                continue
            # when stage is chosen: later stages final, earlier ones initial
            state = np.concatenate([start[:, :stage], final[:, stage:]], axis=1)
            obj = _stage_objective(x, [t[h] for t in tabs_all], state, stage, aff)
            order = np.sort(obj, axis=1)
            clear = (order[:, 1] - order[:, 0]) > 1e-4 * np.maximum(order[:, 0], 1e-6)
            assert np.array_equal(obj.argmin(1)[clear], final[clear, stage]), f"stage {stage} head {h}"
            checked += int(clear.sum())
    assert checked > 150


def test_oracle_objective_never_rises():
    states, tables, init = _problem(11, 2, 2, 64, 8, 32, 4)
    _out, _idx, hist, initial = ora.coordinate_refinement(states.numpy(), [t.numpy() for t in tables],
                                                          init.numpy(), (1, 2, 4), (1.0, 1.0, 3.0), sweeps=3)
    seq = [initial] + hist
    assert all(b <= a * (1 + 1e-6) for a, b in zip(seq, seq[1:])), seq
    assert seq[-1] < 0.9 * seq[0]


def test_oracle_nearest_against_float64():
    gen = torch.Generator().manual_seed(3)
    x, c = torch.randn(300, 16, generator=gen), torch.randn(50, 16, generator=gen)
    got = ora.nearest(x.numpy(), c.numpy())
    d = torch.cdist(x.double(), c.double())
    assert np.array_equal(got, d.argmin(1).numpy())
    # ties go to the lowest index
    assert ora.nearest(np.zeros((1, 4), np.float32), np.zeros((3, 4), np.float32))[0] == 0


@pytest.mark.parametrize("kwargs,match", [
    (dict(prefixes=(), exit_weights=()), "prefixes must lie"),
    (dict(prefixes=(4,), exit_weights=(1.0,)), "prefixes must lie"),
    (dict(prefixes=(1, 2), exit_weights=(1.0,)), "one finite non-negative weight"),
    (dict(prefixes=(1,), exit_weights=(0.0,)), "at least one exit weight"),
    (dict(prefixes=(1,), exit_weights=(1.0,), sweeps=0), "sweeps and token chunks"),
])
def test_refinement_argument_errors(kwargs, match):
    states, tables, init = _problem(1, 1, 2, 8, 4, 8, 3)
    with pytest.raises(ValueError, match=match):
        jkv.multi_exit_additive_coordinate_refinement(states, tables, init, **kwargs)


def test_refinement_rejects_bad_indices():
    states, tables, init = _problem(1, 1, 2, 8, 4, 8, 2)
    with pytest.raises(ValueError, match="initial indices differ"):
        jkv.multi_exit_additive_coordinate_refinement(states, tables, init[..., :1], prefixes=(2,),
                                                      exit_weights=(1.0,))
    init[0, 0, 0, 1] = 8
    with pytest.raises(ValueError, match="outside its codebook"):
        jkv.multi_exit_additive_coordinate_refinement(states, tables, init, prefixes=(2,), exit_weights=(1.0,))


@pytest.mark.gpu
@pytest.mark.parametrize("heads,rows,dim,clusters", [(3, 1000, 128, 256), (2, 77, 7, 100), (1, 64, 128, 64)])
def test_nearest_f32_matches_oracle(device, heads, rows, dim, clusters):
    print(f"nearest H={heads} N={rows} D={dim} K={clusters}", flush=True)
    gen = torch.Generator().manual_seed(rows + dim)
    x = torch.randn(heads, rows, dim, generator=gen)
    c = torch.randn(heads, clusters, dim, generator=gen)
    got = _ops.nearest_f32(x.to(device), c.to(device)).cpu().numpy()
    for h in range(heads):
        want = ora.nearest(x[h].numpy(), c[h].numpy())
        d = np.sort(torch.cdist(x[h].double(), c[h].double()).square().numpy(), axis=1)
        clear = (d[:, 1] - d[:, 0]) > 1e-3 * d[:, 0]
        assert np.array_equal(got[h][clear], want[clear])
        assert (got[h] == want).mean() >= 0.9999


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,batch,tokens,sweeps", [(torch.float32, 2, 300, 2), (torch.float16, 1, 65, 1)])
def test_refinement_matches_oracle(device, dtype, batch, tokens, sweeps):
    print(f"refinement dtype={dtype} B={batch} T={tokens} sweeps={sweeps}", flush=True)
    states, tables, init = _problem(23 + tokens, batch, 4, tokens, 128, 256, 3)
    states = states.to(dtype)
    prefixes, weights = (1, 2, 3), (1.0, 1.0, 2.0)
    out, idx, diag = jkv.multi_exit_additive_coordinate_refinement(
        states.to(device), [t.to(device) for t in tables], init.to(device), prefixes=prefixes,
        exit_weights=weights, sweeps=sweeps)
    r_out, r_idx, r_hist, r_init = ora.coordinate_refinement(states.float().numpy(), [t.numpy() for t in tables],
                                                             init.numpy(), prefixes, weights, sweeps=sweeps)
    assert idx.dtype == torch.uint8 and tuple(idx.shape) == (batch, 4, tokens, 3)
    same = (idx.cpu().long().numpy() == r_idx).all(-1)
    assert same.mean() >= 0.999, same.mean()
    for p in prefixes:
        assert out[p].dtype == dtype
        err = np.abs(out[p].cpu().float().numpy() - r_out[p].astype(np.float32).astype(
            np.float16 if dtype == torch.float16 else np.float32).astype(np.float32))[same].max()
        assert err <= 1e-4, (p, err)
    assert diag["final_weighted_objective"] == pytest.approx(r_hist[-1], rel=1e-4)
    assert diag["initial_weighted_objective"] == pytest.approx(r_init, rel=1e-5)
    assert diag["final_weighted_objective"] < diag["initial_weighted_objective"]
    assert len(diag["sweep_history"]) == sweeps and diag["mode"] == "multi_exit_additive_coordinate"


def test_oracle_topk_against_float64_sort():
    gen = torch.Generator().manual_seed(5)
    x, c = torch.randn(200, 12, generator=gen), torch.randn(40, 12, generator=gen)
    excl = torch.randint(0, 40, (200,), generator=gen).numpy()
    got = ora.nearest_topk(x.numpy(), c.numpy(), 5, excl)
    d = torch.cdist(x.double(), c.double()).numpy()
    d[np.arange(200), excl] = np.inf
    assert np.array_equal(got, np.argsort(d, axis=1, kind="stable")[:, :5])
    assert not (got == excl[:, None]).any()


def test_block_oracle_with_full_shortlist_is_the_exhaustive_pair_optimum():
    # two stages, one block; a shortlist of every codeword makes the block
    # step the joint optimum over all K^2 pairs
    states, tables, init = _problem(9, 1, 2, 30, 5, 6, 2)
    prefixes, weights = (1, 2), (1.0, 2.0)
    _out, idx, hist, initial = ora.block_refinement(states.numpy(), [t.numpy() for t in tables], init.numpy(),
                                                    prefixes, weights, sweeps=1, shortlist=6)
    assert hist[0] <= initial
    checked = 0
    for h in range(2):
        x = states[0, h].double().numpy()
        t0, t1 = tables[0][h].double().numpy(), tables[1][h].double().numpy()
        e1 = np.square(x[:, None, :] - t0[None]).sum(-1)                               # [N, K]
        e2 = np.square(x[:, None, None, :] - t0[None, :, None] - t1[None, None]).sum(-1)  # [N, K, K]
        cost = (weights[0] * e1[:, :, None] + weights[1] * e2).reshape(len(x), -1)
        order = np.sort(cost, axis=1)
        clear = (order[:, 1] - order[:, 0]) > 1e-4 * np.maximum(order[:, 0], 1e-6)
        best = cost.argmin(1)
        assert np.array_equal((best // 6)[clear], idx[0, h, clear, 0])
        assert np.array_equal((best % 6)[clear], idx[0, h, clear, 1])
        checked += int(clear.sum())
    assert checked > 40


def test_block_oracle_objective_never_rises():
    states, tables, init = _problem(13, 1, 2, 30, 8, 16, 3)
    _out, _idx, hist, initial = ora.block_refinement(states.numpy(), [t.numpy() for t in tables], init.numpy(),
                                                     (1, 2, 3), (1.0, 1.0, 2.0), sweeps=2, shortlist=3)
    seq = [initial] + hist
    assert all(b <= a * (1 + 1e-6) for a, b in zip(seq, seq[1:])), seq


@pytest.mark.parametrize("kwargs,match", [
    (dict(prefixes=(1,), exit_weights=(1.0,)), "requires at least two stages"),
    (dict(prefixes=(2,), exit_weights=(1.0,), shortlist_size=1), "invalid block-refinement"),
    (dict(prefixes=(2,), exit_weights=(1.0,), shortlist_size=9), "cannot support the requested shortlist"),
])
def test_block_refinement_argument_errors(kwargs, match):
    states, tables, init = _problem(1, 1, 2, 8, 4, 8, 2)
    if kwargs["prefixes"] == (1,):
        init = init[..., :1]
    with pytest.raises(ValueError, match=match):
        jkv.multi_exit_additive_block_refinement(states, tables, init, **kwargs)


@pytest.mark.gpu
@pytest.mark.parametrize("heads,rows,dim,clusters,m,exclude", [(2, 500, 128, 256, 3, True), (1, 70, 9, 40, 8, False),
                                                                (2, 64, 128, 64, 1, True)])
def test_nearest_topk_f32_matches_float64(device, heads, rows, dim, clusters, m, exclude):
    print(f"topk H={heads} N={rows} D={dim} K={clusters} M={m} exclude={exclude}", flush=True)
    gen = torch.Generator().manual_seed(rows + m)
    x = torch.randn(heads, rows, dim, generator=gen)
    c = torch.randn(heads, clusters, dim, generator=gen)
    excl = torch.randint(0, clusters, (heads, rows), generator=gen) if exclude else None
    got = _ops.nearest_topk_f32(x.to(device), c.to(device), m,
                                excluded=None if excl is None else excl.to(device)).cpu().numpy()
    agree = 0
    for h in range(heads):
        want = ora.nearest_topk(x[h].numpy(), c[h].numpy(), m, None if excl is None else excl[h].numpy())
        d = torch.cdist(x[h].double(), c[h].double()).square().numpy()
        if excl is not None:
            d[np.arange(rows), excl[h].numpy()] = np.inf
        ds = np.sort(d, axis=1)[:, :m + 1]
        clear = ((ds[:, 1:] - ds[:, :-1]) > 1e-3 * ds[:, :1]).all(1)
        assert np.array_equal(got[h][clear], np.argsort(d, axis=1, kind="stable")[clear, :m])
        agree += int((got[h] == want).all(1).sum())
    assert agree >= 0.999 * heads * rows


@pytest.mark.gpu
def test_block_refinement_matches_oracle(device):
    print("block refinement H=2 T=100 D=128 K=64 S=3", flush=True)
    states, tables, init = _problem(31, 1, 2, 100, 128, 64, 3)
    prefixes, weights = (1, 2, 3), (1.0, 1.0, 2.0)
    out, idx, diag = jkv.multi_exit_additive_block_refinement(
        states.to(device), [t.to(device) for t in tables], init.to(device), prefixes=prefixes,
        exit_weights=weights, sweeps=1, shortlist_size=4, token_chunk_size=64)
    r_out, r_idx, r_hist, r_init = ora.block_refinement(states.numpy(), [t.numpy() for t in tables], init.numpy(),
                                                        prefixes, weights, sweeps=1, shortlist=4)
    same = (idx.cpu().long().numpy() == r_idx).all(-1)
    assert same.mean() >= 0.99, same.mean()
    for p in prefixes:
        err = np.abs(out[p].cpu().numpy() - r_out[p])[same].max()
        assert err <= 1e-4, (p, err)
    assert diag["final_weighted_objective"] == pytest.approx(r_hist[-1], rel=1e-3)
    assert diag["final_weighted_objective"] <= diag["initial_weighted_objective"]
    assert diag["mode"] == "multi_exit_additive_block" and len(diag["sweep_history"][0]["blocks"]) == 2


@pytest.mark.gpu
@pytest.mark.parametrize("block", [False, True])
def test_zero_weight_exit_keeps_its_initial_reconstruction(device, block):
    # only weighted exits move (nested_vq.py:711-716, :945-948): exit 2 of
    # weight 0 keeps the decode of the initial indices while its stages change
    print(f"zero-weight exit, block={block}", flush=True)
    states, tables, init = _problem(41, 1, 2, 120, 16, 32, 3)
    prefixes, weights = (1, 2, 3), (1.0, 0.0, 2.0)
    args = (states.to(device), [t.to(device) for t in tables], init.to(device))
    if block:
        out, idx, diag = jkv.multi_exit_additive_block_refinement(*args, prefixes=prefixes, exit_weights=weights,
                                                                  shortlist_size=3)
        r_out, r_idx, r_hist, _ = ora.block_refinement(states.numpy(), [t.numpy() for t in tables], init.numpy(),
                                                       prefixes, weights, shortlist=3)
    else:
        out, idx, diag = jkv.multi_exit_additive_coordinate_refinement(*args, prefixes=prefixes, exit_weights=weights)
        r_out, r_idx, r_hist, _ = ora.coordinate_refinement(states.numpy(), [t.numpy() for t in tables],
                                                            init.numpy(), prefixes, weights)
    same = (idx.cpu().long().numpy() == r_idx).all(-1)
    assert same.mean() >= 0.99
    assert (idx.cpu().long() != init).any(), "the sweep moved no index"
    initial_decode = sum(tables[s][torch.arange(2)[None, :, None], init[..., s]] for s in range(2)).permute(0, 1, 2, 3)
    torch.testing.assert_close(out[2].cpu(), initial_decode, rtol=0, atol=1e-6)
    for p in (1, 3):
        assert np.abs(out[p].cpu().numpy() - r_out[p])[same].max() <= 1e-4
    assert diag["final_weighted_objective"] == pytest.approx(r_hist[-1], rel=1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("block", [False, True])
def test_token_chunk_size_changes_nothing(device, block):
    # rows are independent and no step materialises per-chunk temporaries, so
    # the chunk size (validated, as the reference's) must not move a bit
    print(f"chunk independence, block={block}", flush=True)
    states, tables, init = _problem(43, 1, 2, 200, 32, 64, 3)
    runs = []
    for chunk in (1, 64, 4096):
        args = (states.to(device), [t.to(device) for t in tables], init.to(device))
        fn = jkv.multi_exit_additive_block_refinement if block else jkv.multi_exit_additive_coordinate_refinement
        out, idx, diag = fn(*args, prefixes=(1, 2, 3), exit_weights=(1.0, 1.0, 2.0), sweeps=2, token_chunk_size=chunk)
        runs.append((out, idx, diag["final_weighted_objective"]))
    for out, idx, obj in runs[1:]:
        assert torch.equal(idx, runs[0][1])
        for p in (1, 2, 3):
            assert torch.equal(out[p], runs[0][0][p])
        assert obj == runs[0][2]


@pytest.mark.gpu
@pytest.mark.parametrize("dim,clusters,shortlist", [(7, 40, 4), (128, 64, 9), (16, 256, 2)])
def test_block_refinement_kernel_paths_match_oracle(device, dim, clusters, shortlist):
    # odd D takes the scalar scoring loop, shortlist 9 gives lanes two pairs
    print(f"block kernel D={dim} K={clusters} L={shortlist}", flush=True)
    states, tables, init = _problem(47 + dim, 1, 2, 90, dim, clusters, 3)
    prefixes, weights = (2, 3), (1.0, 3.0)
    out, idx, diag = jkv.multi_exit_additive_block_refinement(
        states.to(device), [t.to(device) for t in tables], init.to(device), prefixes=prefixes, exit_weights=weights,
        shortlist_size=shortlist)
    r_out, r_idx, r_hist, r_init = ora.block_refinement(states.numpy(), [t.numpy() for t in tables], init.numpy(),
                                                        prefixes, weights, shortlist=shortlist)
    same = (idx.cpu().long().numpy() == r_idx).all(-1)
    assert same.mean() >= 0.98, same.mean()
    for p in prefixes:
        assert np.abs(out[p].cpu().numpy() - r_out[p])[same].max() <= 1e-4
    assert diag["final_weighted_objective"] <= diag["initial_weighted_objective"] * (1 + 1e-6)
    assert diag["final_weighted_objective"] == pytest.approx(r_hist[-1], rel=1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("block", [False, True])
def test_refinement_leaves_its_inputs_alone(device, block):
    # batch 1 makes the permuted index view contiguous: the sweep must still
    # work on a copy of the caller's indices (and states, tables)
    states, tables, init = _problem(53, 1, 2, 64, 16, 32, 2)
    args = [states.to(device), [t.to(device) for t in tables], init.to(device)]
    before = [args[0].clone(), [t.clone() for t in args[1]], args[2].clone()]
    fn = jkv.multi_exit_additive_block_refinement if block else jkv.multi_exit_additive_coordinate_refinement
    _out, idx, _diag = fn(*args, prefixes=(1, 2), exit_weights=(1.0, 1.0))
    assert (idx.cpu().long() != init).any()
    assert torch.equal(args[0], before[0]) and torch.equal(args[2], before[2])
    assert all(torch.equal(a, b) for a, b in zip(args[1], before[1]))
