"""Encode parity on the MI355X: HIP kernels vs the CPU oracle."""

from __future__ import annotations

import pytest
import torch

import jointkv_amd as jkv
from oracle import jointkv_oracle as ref

from parity import assert_codes, assert_codes_with_exact_floor, assert_recon_rows, bruteforce_rvq_codes

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def test_config1_grouped_cq_full_size(device):
    # [1,8,2048,128] fp16 with 4 outlier channels per head,
    # codebooks [8,16,256,8] N(0,1), seed 8601 (K then V).
    gen = _gen(8601)
    key = ref.synthetic_states(gen, 1, 8, 2048)
    value = ref.synthetic_states(gen, 1, 8, 2048)
    kbook = ref.synthetic_tables(gen, (8, 16, 256, 8), (1.0,), stage_axis=0)
    vbook = ref.synthetic_tables(gen, (8, 16, 256, 8), (1.0,), stage_axis=0)
    for states, books in ((key, kbook), (value, vbook)):
        print(f"config1 grouped CQ {tuple(states.shape)} x {tuple(books.shape)}", flush=True)
        out, codes = jkv.hard_grouped_cq(states.to(device), books.to(device))
        r_out, r_codes, d1, d2 = ref.hard_grouped_cq(states, books, return_margins=True)
        res = assert_codes(codes[..., None], r_codes[..., None], d1[..., None], d2[..., None])
        rows = (codes.cpu() == r_codes)
        # per-group rows: compare 8-dim slices
        o = out.cpu().reshape(1, 8, 2048, 16, 8)
        r = r_out.detach().reshape(1, 8, 2048, 16, 8)
        assert_recon_rows(o, r, rows)
        assert codes.dtype == torch.uint8 and codes.shape == (1, 8, 2048, 16)
        assert res["agreement"] >= 0.9999


# (1500, 3): 4500 rows per problem give workgroups two 256-row iterations
# each, with batch boundaries inside iterations and a ragged last chunk
@pytest.mark.parametrize("tokens,batch", [(512, 1), (300, 2), (1500, 3)])
def test_grouped_residual_two_stage(device, tokens, batch):
    # G2 geometry of BASELINE config 2 (16 groups x 8 dims, 2 stages, s2 sigma 0.5)
    gen = _gen(8601 + tokens)
    states = ref.synthetic_states(gen, batch, 8, tokens)
    tables = ref.synthetic_tables(gen, (8, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2)
    print(f"G2 encode B={batch} T={tokens}", flush=True)
    exits, codes = jkv.hard_grouped_residual_vq(states.to(device), tables.to(device), prefixes=(1, 2))
    r_exits, r_codes, d1, d2 = ref.grouped_residual_vq(states, tables, prefixes=(1, 2), return_margins=True)
    res = assert_codes(codes, r_codes, d1, d2)
    for depth in (1, 2):
        o = exits[depth].cpu().reshape(batch, 8, tokens, 16, 8)
        r = r_exits[depth].detach().reshape(batch, 8, tokens, 16, 8)
        assert_recon_rows(o, r, res["prefix_ok"])


# (2, 256): one iteration per workgroup; (4, 2048): BASELINE config 3's
# [4,8,2048,128], four 256-row iterations per workgroup
@pytest.mark.parametrize("batch,tokens", [(2, 256), (4, 2048)])
def test_cq2_geometry_d4(device, batch, tokens):
    # reference cq2 cell: [8,32,256,4] (BASELINE config 3 geometry)
    gen = _gen(8602)
    states = ref.synthetic_states(gen, batch, 8, tokens)
    books = ref.synthetic_tables(gen, (8, 32, 256, 4), (1.0,), stage_axis=0)
    print(f"cq2 encode B={batch} T={tokens}", flush=True)
    out, codes = jkv.hard_grouped_cq(states.to(device), books.to(device))
    r_out, r_codes, d1, d2 = ref.hard_grouped_cq(states, books, return_margins=True)
    res = assert_codes(codes[..., None], r_codes[..., None], d1[..., None], d2[..., None])
    assert_recon_rows(out.cpu().reshape(batch, 8, tokens, 32, 4), r_out.detach().reshape(batch, 8, tokens, 32, 4),
                      codes.cpu() == r_codes)


@pytest.mark.parametrize("seed,dtype,dim,stages,clusters", [
    (7, torch.float32, 4, 3, 4),
    (9, torch.float32, 4, 3, 4),
    (10, torch.float16, 4, 3, 4),
    (43, torch.float32, 3, 2, 8),
    (5, torch.bfloat16, 16, 3, 64),
    (6, torch.float16, 128, 2, 256),
])
def test_residual_vq_generic_geometries(device, seed, dtype, dim, stages, clusters):
    # the reference's own tiny cases (tests/test_closed_loop_vq.py) and wider ones
    gen = _gen(seed)
    states = torch.randn(1, 2, 37, dim, generator=gen).to(dtype)
    tables = torch.randn(2, stages, clusters, dim, generator=gen)
    prefixes = tuple(range(1, stages + 1))
    exits, codes = jkv.hard_residual_vq_exits(states.to(device), tables.to(device), prefixes=prefixes)
    r_exits, r_codes, d1, d2 = ref.hard_residual_vq_exits(states, tables, prefixes=prefixes,
                                                          return_margins=True)
    res = assert_codes(codes, r_codes, d1, d2, agreement=0.99)
    for depth in prefixes:
        assert exits[depth].dtype == dtype
        assert_recon_rows(exits[depth].cpu(), r_exits[depth].detach(), res["prefix_ok"])


# full-vector codebooks (d = 128, K = 256): the MFMA kernel with fp16-deployed
# tables in the workspace; ragged rows, many stages, exits at several depths
@pytest.mark.parametrize("batch,tokens,stages,prefixes", [
    (1, 300, 2, (1, 2)),
    (2, 77, 4, (2, 4)),
    (1, 40, 16, (1, 8, 16)),
    (1, 64, 32, (16, 32)),   # R32 (gsrq2): the 32-stage maximum
])
def test_full_vector_residual_vq(device, batch, tokens, stages, prefixes):
    gen = _gen(700 + stages)
    states = ref.synthetic_states(gen, batch, 8, tokens)
    tables = ref.synthetic_tables(gen, (8, stages, 256, 128), tuple(0.8 ** s for s in range(stages)), stage_axis=1)
    print(f"full-vector encode B={batch} T={tokens} S={stages}", flush=True)
    exits, codes = jkv.hard_residual_vq_exits(states.to(device), tables.to(device), prefixes=prefixes)
    r_exits, r_codes, d1, d2 = ref.hard_residual_vq_exits(states, tables, prefixes=prefixes, return_margins=True)
    assert_codes_with_exact_floor(codes, r_codes, d1, d2, *bruteforce_rvq_codes(states, tables))
    for depth in prefixes:
        rows = (codes.cpu().long()[..., :depth] == r_codes.long()[..., :depth]).all(-1)
        assert_recon_rows(exits[depth].cpu(), r_exits[depth].detach(), rows)


def test_full_vector_config3_literal(device):
    # the literal reading of BASELINE config 3: [4,8,2048,128] with two
    # full-dim stages [8,2,256,128] (s1 N(0,1), s2 sigma 0.5), every token
    gen = _gen(8601)
    states = ref.synthetic_states(gen, 4, 8, 2048)
    tables = ref.synthetic_tables(gen, (8, 2, 256, 128), (1.0, 0.5), stage_axis=1)
    print("full-vector encode config 3 literal [4,8,2048,128] S=2", flush=True)
    exits, codes = jkv.hard_residual_vq_exits(states.to(device), tables.to(device), prefixes=(2,))
    r_exits, r_codes, d1, d2 = ref.hard_residual_vq_exits(states, tables, prefixes=(2,), return_margins=True)
    res = assert_codes(codes, r_codes, d1, d2)
    assert_recon_rows(exits[2].cpu(), r_exits[2].detach(), res["prefix_ok"])


@pytest.mark.parametrize("seed", [41, 42])
def test_whitened_search(device, seed):
    gen = _gen(seed)
    states = torch.randn(1, 2, 64, 8, generator=gen).half()
    tables = torch.randn(2, 3, 32, 8, generator=gen)
    w = torch.randn(2, 8, 8, generator=gen)
    exits, codes = jkv.hard_residual_vq_exits(states.to(device), tables.to(device), prefixes=(3,),
                                              assignment_whiteners=w.to(device))
    r_exits, r_codes, d1, d2 = ref.hard_residual_vq_exits(states, tables, prefixes=(3,),
                                                          assignment_whiteners=w, return_margins=True)
    res = assert_codes(codes, r_codes, d1, d2, agreement=0.99)
    assert_recon_rows(exits[3].cpu(), r_exits[3].detach(), res["prefix_ok"])
    # grouped CQ with a per-(head, group) selector whitener
    books = torch.randn(2, 4, 256, 2, generator=gen)
    f = torch.randn(2, 4, 2, 2, generator=gen)
    st = torch.randn(1, 2, 64, 8, generator=gen)
    out, c = jkv.hard_grouped_cq(st.to(device), books.to(device), selector_whiteners=f.to(device))
    r_out, r_c, e1, e2 = ref.hard_grouped_cq(st, books, selector_whiteners=f, return_margins=True)
    assert_codes(c[..., None], r_c[..., None], e1[..., None], e2[..., None], agreement=0.99)


@pytest.mark.parametrize("heads,tokens,stages,prefixes", [
    (2, 96, 4, (2, 4)),
    (2, 300, 16, (1, 8, 16)),
    (8, 512, 2, (1, 2)),
    (2, 48, 32, (32,)),
])
def test_whitened_search_full_vector(device, heads, tokens, stages, prefixes):
    # d = 128 assignment whitener (upper triangular, as GSRQ fitting leaves
    # it): the whitened full-vector MFMA kernel
    gen = _gen(43 + stages)
    sig = tuple(0.8 ** s for s in range(stages))
    states = ref.synthetic_states(gen, 1, heads, tokens, 128)
    tables = ref.synthetic_tables(gen, (heads, stages, 256, 128), sig, stage_axis=1)
    w = torch.triu(torch.randn(heads, 128, 128, generator=gen) * 0.1) + torch.eye(128)
    print(f"whitened full-vector H={heads} T={tokens} S={stages}", flush=True)
    exits, codes = jkv.hard_residual_vq_exits(states.to(device), tables.to(device), prefixes=prefixes,
                                              assignment_whiteners=w.to(device))
    r_exits, r_codes, d1, d2 = ref.hard_residual_vq_exits(states, tables, prefixes=prefixes,
                                                          assignment_whiteners=w, return_margins=True)
    assert_codes_with_exact_floor(codes, r_codes, d1, d2, *bruteforce_rvq_codes(states, tables, w))
    for depth in prefixes:
        rows = (codes.cpu().long()[..., :depth] == r_codes.long()[..., :depth]).all(-1)
        assert_recon_rows(exits[depth].cpu(), r_exits[depth].detach(), rows)


def test_edge_cases_empty_ragged_and_ties(device):
    tables = torch.randn(2, 2, 256, 8)
    # empty token axis
    exits, codes = jkv.hard_grouped_residual_vq(torch.zeros(1, 2, 0, 16, dtype=torch.float16, device=device),
                                                tables.reshape(2, 1, 2, 256, 8).expand(2, 2, 2, 256, 8).contiguous().to(device),
                                                prefixes=(2,))
    assert codes.shape == (1, 2, 0, 2, 2) and exits[2].shape == (1, 2, 0, 16)
    # ragged tile: 17 rows; duplicated codewords -> lowest index wins (argmin)
    dup = torch.randn(1, 1, 256, 8)
    dup[0, 0, 200] = dup[0, 0, 3]
    states = dup[0, 0, 3].repeat(1, 1, 17, 1).half()
    exits, codes = jkv.hard_residual_vq_exits(states.to(device), dup.to(device), prefixes=(1,))
    assert bool((codes.cpu() == 3).all())
    # non-contiguous states view (strided heads)
    base = ref.synthetic_states(_gen(3), 1, 4, 33)
    view = base[:, ::2]
    t = ref.synthetic_tables(_gen(4), (2, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2)
    e1, c1 = jkv.hard_grouped_residual_vq(view.to(device), t.to(device), prefixes=(2,))
    e2, c2 = jkv.hard_grouped_residual_vq(view.contiguous().to(device), t.to(device), prefixes=(2,))
    assert torch.equal(c1, c2) and torch.equal(e1[2], e2[2])


def test_inputs_are_not_mutated(device):
    gen = _gen(170817)
    states = ref.synthetic_states(gen, 1, 2, 64).to(device)
    tables = ref.synthetic_tables(gen, (2, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2).to(device)
    s0, t0 = states.clone(), tables.clone()
    jkv.hard_grouped_residual_vq(states, tables, prefixes=(2,))
    assert torch.equal(states, s0) and torch.equal(tables, t0)


@pytest.mark.parametrize("heads,groups,d,stages,depth,clusters,dtype,cap", [
    (2, 16, 8, 2, 2, 256, torch.float16, None),   # GSRQ-2: one 16-byte output per group
    (2, 16, 8, 2, 1, 256, torch.bfloat16, 40),    # first stage only, codes as a code-cache slice
    (1, 8, 16, 3, 3, 64, torch.float32, None),    # two 8-wide chunks per group, fp32 out
    (2, 4, 4, 2, 2, 16, torch.float16, None),     # 4-wide chunks
    (1, 5, 3, 2, 2, 7, torch.float32, None),      # odd width: one output at a time
])
def test_rvq_decode_matches_oracle(device, heads, groups, d, stages, depth, clusters, dtype, cap):
    # the frozen-code decode, bit for bit: fp32 sum of the fp16-deployed
    # words in stage order, one cast at the end
    print(f"rvq_decode H={heads} G={groups} d={d} S={stages} depth={depth} K={clusters} {dtype} cap={cap}",
          flush=True)
    gen = _gen(4242 + d)
    batch, tokens = 2, 33
    tables = ref.synthetic_tables(gen, (heads * groups, stages, clusters, d), (1.0, 0.5, 0.25)[:stages],
                                  stage_axis=1)
    # fp32 masters off the fp16 grid, so that the deploy rounding matters
    tables = tables + 1e-3 * torch.randn(tables.shape, generator=gen)
    codes = torch.randint(0, clusters, (batch, heads, cap or tokens, groups, stages), generator=gen,
                          dtype=torch.uint8)[:, :, :tokens]
    got = jkv.closed_loop_vq._ops.rvq_decode(codes.to(device), tables.to(device), depth=depth, dtype=dtype)
    want = ref.frozen_decode(codes.contiguous(), tables, depth, dtype)
    assert got.dtype == dtype and torch.equal(got.cpu(), want)


def test_full_size_layer_properties(device):
    # BASELINE config 2 at full per-layer size: [1,8,8192,128], G2 tables.
    gen = _gen(8601)
    states = ref.synthetic_states(gen, 1, 8, 8192).to(device)
    tables = ref.synthetic_tables(gen, (8, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2).to(device)
    exits, codes = jkv.hard_grouped_residual_vq(states, tables, prefixes=(1, 2))
    # exits equal the frozen decode of the codes (two independent kernels)
    flat = tables.reshape(128, 2, 256, 8)
    for depth in (1, 2):
        dec = jkv.closed_loop_vq._ops.rvq_decode(codes, flat, depth=depth, dtype=torch.float16)
        assert torch.equal(dec, exits[depth])
    # every token checked against the oracle (workgroups here run four
    # 256-row iterations, so this covers rows past the first iteration)
    r_exits, r_codes, d1, d2 = ref.grouped_residual_vq(states.cpu(), tables.cpu(), prefixes=(2,),
                                                       return_margins=True)
    res = assert_codes(codes, r_codes, d1, d2)
    assert_recon_rows(exits[2].cpu().reshape(1, 8, 8192, 16, 8), r_exits[2].detach().reshape(1, 8, 8192, 16, 8),
                      res["prefix_ok"])
    # stage-1 optimality: the chosen word is at least as close (fp64) as every other
    x = states[0, :, :64].float().reshape(8, 64, 16, 8).cpu().double()
    c1 = tables[:, :, 0].cpu().double()  # [8,16,256,8]
    dist = ((x[:, :, :, None, :] - c1[:, None]) ** 2).sum(-1)  # [8,64,16,256]
    chosen = dist.gather(-1, codes[0, :, :64, :, 0].long().cpu()[..., None])[..., 0]
    best = dist.min(-1).values
    assert bool(((chosen - best) <= 1e-3 * best.clamp_min(1e-9)).all())


@pytest.mark.parametrize("batch,tokens,groups,dim,stages,dtype,exits", [
    (2, 300, 16, 8, 2, torch.float16, (1, 2)),     # G2: one paired launch
    (16, 1, 32, 4, 1, torch.float16, (1,)),        # cq2, one token per sequence (the decode step)
    (1, 70, 16, 8, 2, torch.float32, (2,)),        # fp32 states: the two encodes in turn
    (1, 40, 1, 128, 4, torch.float16, (2, 4)),     # full-vector tables: in turn, shared workspace
])
def test_encode_kv_equals_two_encodes(device, batch, tokens, groups, dim, stages, dtype, exits):
    from jointkv_amd import _ops

    print(f"encode_kv B={batch} T={tokens} G={groups} d={dim} S={stages} {dtype}", flush=True)
    gen = _gen(4242 + tokens)
    k = ref.synthetic_states(gen, batch, 8, tokens, groups * dim).to(dtype).to(device)
    v = ref.synthetic_states(gen, batch, 8, tokens, groups * dim).to(dtype).to(device)
    sig = tuple(0.5 ** s for s in range(stages))
    kt = ref.synthetic_tables(gen, (8 * groups, stages, 256, dim), sig, stage_axis=1).to(device)
    vt = ref.synthetic_tables(gen, (8 * groups, stages, 256, dim), sig, stage_axis=1).to(device)
    rk, ck, rv, cv = _ops.rvq_encode_kv(k, v, kt, vt, groups=groups, group_dim=dim, exits=exits)
    ek, eck = _ops.rvq_encode(k, kt, groups=groups, group_dim=dim, exits=exits)
    ev, ecv = _ops.rvq_encode(v, vt, groups=groups, group_dim=dim, exits=exits)
    assert torch.equal(ck, eck) and torch.equal(cv, ecv)
    for a, b in zip(rk + rv, ek + ev):
        assert torch.equal(a, b)


# (heads, batch, tokens, groups, dim, stages, dtype, exits, jobs)
@pytest.mark.parametrize("heads,batch,tokens,groups,dim,stages,dtype,exits,jobs", [
    (8, 2, 300, 16, 8, 2, torch.float16, (1, 2), 5),    # G2, one launch, ragged rows
    # 70 jobs: a 64-job launch whose workgroups take 4,096-row ranges (16
    # iterations per wave, a ragged second chunk), then a 6-job launch
    (2, 1, 4500, 16, 8, 2, torch.float16, (2,), 70),
    (8, 16, 1, 32, 4, 1, torch.float16, (1,), 4),       # cq2, one token per sequence
    (8, 1, 70, 16, 8, 2, torch.float32, (2,), 3),       # fp32 states: the encodes in turn
    (8, 1, 40, 1, 128, 4, torch.float16, (2, 4), 2),    # full-vector tables: one table launch, one search launch
    (8, 2, 300, 1, 128, 2, torch.float16, (1, 2), 5),    # full-vector, config-3-like: both tables kept for a run
    (8, 1, 700, 1, 128, 16, torch.float16, (8, 16), 3),  # full-vector, 16 stages streamed through a run
    (8, 1, 50, 1, 128, 4, torch.float16, (1, 2, 4), 2),  # full-vector with three exits: one encode per job
    (2, 1, 40, 1, 128, 2, torch.float16, (2,), 66),     # full-vector, 64 + 2 jobs: the workspace regions reused
])
def test_encode_many_equals_per_job_encodes(device, heads, batch, tokens, groups, dim, stages, dtype, exits, jobs):
    from jointkv_amd import _ops

    print(f"encode_many jobs={jobs} H={heads} B={batch} T={tokens} G={groups} d={dim} S={stages} {dtype}",
          flush=True)
    gen = _gen(5150 + tokens + jobs)
    sig = tuple(0.5 ** s for s in range(stages))
    states_cpu = [ref.synthetic_states(gen, batch, heads, tokens, groups * dim) for _ in range(jobs)]
    tables_cpu = [ref.synthetic_tables(gen, (heads * groups, stages, 256, dim), sig, stage_axis=1)
                  for _ in range(jobs)]
    states = [x.to(dtype).to(device) for x in states_cpu]
    tables = [t.to(device) for t in tables_cpu]
    out = _ops.rvq_encode_many(states, tables, groups=groups, group_dim=dim, exits=exits)
    assert len(out) == jobs
    for j, (recon, codes) in enumerate(out):
        e_recon, e_codes = _ops.rvq_encode(states[j], tables[j], groups=groups, group_dim=dim, exits=exits)
        assert torch.equal(codes, e_codes), f"job {j}: codes differ from its own encode"
        for a, b in zip(recon, e_recon):
            assert torch.equal(a, b), f"job {j}: reconstructions differ from its own encode"
    if dtype == torch.float16 and dim == 8 and stages == 2 and batch * tokens <= 600:
        # the last job against the oracle as well
        st = states_cpu[-1].half()
        r_exits, r_codes, d1, d2 = ref.grouped_residual_vq(
            st, tables_cpu[-1].reshape(heads, groups, stages, 256, dim), prefixes=(1, 2), return_margins=True)
        assert_codes(out[-1][1], r_codes, d1, d2)
    assert _ops.rvq_encode_many([], [], groups=groups, group_dim=dim, exits=exits) == []


@pytest.mark.parametrize("dim,batch,tokens,seed", [(4, 2, 300, 51), (4, 4, 2048, 52), (4, 16, 1, 53),
                                                    (8, 2, 300, 54), (8, 1, 2048, 55), (8, 16, 1, 56)])
def test_whitened_grouped_cq_on_mfma(device, dim, batch, tokens, seed):
    # the cq2 cell [8,32,256,4] and the cq1 cell [8,16,256,8] with
    # per-(head, group) selector whiteners: the MFMA kernel with M = F^T F
    # (codes at clear margins exact, recon equal wherever codes agree)
    print(f"whitened cq d={dim} B={batch} T={tokens}", flush=True)
    gen = _gen(seed)
    states = ref.synthetic_states(gen, batch, 8, tokens)
    books = ref.synthetic_tables(gen, (8, 128 // dim, 256, dim), (1.0,), stage_axis=0)
    f = torch.eye(dim) + 0.3 * torch.randn(8, 128 // dim, dim, dim, generator=gen)
    out, codes = jkv.hard_grouped_cq(states.to(device), books.to(device), selector_whiteners=f.to(device))
    r_out, r_codes, d1, d2 = ref.hard_grouped_cq(states, books, selector_whiteners=f, return_margins=True)
    res = assert_codes(codes[..., None], r_codes[..., None], d1[..., None], d2[..., None])
    rows = res["prefix_ok"].all(-1)
    same = (codes.cpu() == r_codes).all(-1)
    assert torch.equal(out.cpu()[same], r_out.detach()[same])


def test_encode_many_full_cache_equals_per_layer_launches(device):
    # the bench's headline workload at full size: the 64 tensors of a
    # 32-layer [1,8,8192,128] G2 cache in one call, against each layer's
    # K/V launch (itself checked against the oracle above), bit for bit
    from jointkv_amd import _ops

    print("encode_many full config-2 cache (64 x [1,8,8192,128])", flush=True)
    gen = torch.Generator(device=device).manual_seed(8601)
    states = [(torch.randn(1, 8, 8192, 128, generator=gen, device=device)).half() for _ in range(64)]
    tables = [(torch.randn(128, 2, 256, 8, generator=gen, device=device)
               * torch.tensor([1.0, 0.5], device=device)[None, :, None, None]).half().float() for _ in range(64)]
    out = _ops.rvq_encode_many(states, tables, groups=16, group_dim=8, exits=(1, 2))
    for layer in range(32):
        k, v = 2 * layer, 2 * layer + 1
        rk, ck, rv, cv = _ops.rvq_encode_kv(states[k], states[v], tables[k], tables[v], groups=16, group_dim=8,
                                            exits=(1, 2))
        assert torch.equal(out[k][1], ck) and torch.equal(out[v][1], cv), f"layer {layer}: codes"
        for a, b in zip(out[k][0] + out[v][0], rk + rv):
            assert torch.equal(a, b), f"layer {layer}: reconstructions"


def test_encode_many_strided_views_and_geometry_errors(device):
    # states given as [B,T,H,D] storage viewed as [B,H,T,D] (the layout a
    # projection produces), mixed with contiguous ones: each job's output
    # equals its own encode; mismatched geometry is refused
    from jointkv_amd import _ops

    gen = torch.Generator(device=device).manual_seed(5161)
    base = [torch.randn(2, 300, 8, 128, generator=gen, device=device).half() for _ in range(3)]
    states = [base[0].transpose(1, 2), base[1].transpose(1, 2).contiguous(), base[2].transpose(1, 2)]
    tables = [(torch.randn(128, 2, 256, 8, generator=gen, device=device)).half().float() for _ in range(3)]
    out = _ops.rvq_encode_many(states, tables, groups=16, group_dim=8, exits=(2,))
    for j in range(3):
        recon, codes = _ops.rvq_encode(states[j], tables[j], groups=16, group_dim=8, exits=(2,))
        assert torch.equal(out[j][1], codes) and torch.equal(out[j][0][0], recon[0]), f"job {j}"
    with pytest.raises(ValueError, match="geometry"):
        _ops.rvq_encode_many([states[0], states[1][:, :, :200]], tables[:2], groups=16, group_dim=8, exits=(2,))
    with pytest.raises(ValueError):
        _ops.rvq_encode_many(states[:2], tables[:1], groups=16, group_dim=8, exits=(2,))


def test_encode_many_full_vector_config3_literal_equals_per_tensor(device):
    # config 3 read as two full-vector stages at full size: 64 tensors
    # [4,8,2048,128] with tables [8,2,256,128] in one call, against each
    # tensor's own encode (itself checked against the oracle), bit for bit
    from jointkv_amd import _ops

    print("encode_many full-vector config 3 (64 x [4,8,2048,128], S = 2)", flush=True)
    gen = torch.Generator(device=device).manual_seed(8602)
    states = [torch.randn(4, 8, 2048, 128, generator=gen, device=device).half() for _ in range(64)]
    tables = [(torch.randn(8, 2, 256, 128, generator=gen, device=device)
               * torch.tensor([1.0, 0.5], device=device)[None, :, None, None]).half().float() for _ in range(64)]
    out = _ops.rvq_encode_many(states, tables, groups=1, group_dim=128, exits=(2,))
    for j in range(64):
        recon, codes = _ops.rvq_encode(states[j], tables[j], groups=1, group_dim=128, exits=(2,))
        assert torch.equal(out[j][1], codes) and torch.equal(out[j][0][0], recon[0]), f"tensor {j}"


@pytest.mark.parametrize("groups,d,stages,depth,dtype", [
    (16, 8, 2, 2, torch.float16),     # the GSRQ-2 cache geometry (8-element chunks)
    (32, 4, 1, 1, torch.float16),     # grouped CQ (4-element chunks)
    (1, 128, 4, 3, torch.float32),    # full-vector, fp32 out
    (4, 6, 2, 2, torch.bfloat16),     # d = 6: element-wise
])
def test_rvq_decode_from_fp16_tables_equals_masters(device, groups, d, stages, depth, dtype):
    # the deployed fp16 words give the same reconstruction as the fp32 masters
    # (which the kernel rounds to fp16 itself), bit for bit
    from jointkv_amd import _ops

    gen = torch.Generator(device=device).manual_seed(3300 + groups + d)
    codes = torch.randint(0, 256, (2, 8, 77, groups, stages), generator=gen, device=device,
                          dtype=torch.int32).to(torch.uint8)
    masters = torch.randn(8 * groups, stages, 256, d, generator=gen, device=device)
    a = _ops.rvq_decode(codes, masters, depth=depth, dtype=dtype)
    b = _ops.rvq_decode(codes, masters.half(), depth=depth, dtype=dtype)
    assert torch.equal(a, b)


@pytest.mark.parametrize("groups,stages,depth,tables_f16,dtype", [
    (16, 2, 2, False, torch.float16),   # GSRQ-2 masters: two 512-token runs and a ragged third
    (16, 2, 1, True, torch.float32),    # deployed fp16 words, first stage only
    (32, 1, 1, True, torch.bfloat16),   # grouped CQ's 32 x 8 cell (G S = 32)
])
def test_rvq_decode_lds_runs_match_oracle(device, groups, stages, depth, tables_f16, dtype):
    # 8-dim groups rebuild from tables staged in LDS, 512 tokens per
    # workgroup: bit for bit against the oracle over several runs per head
    gen = _gen(6161 + groups + stages)
    batch, heads, tokens = 2, 3, 1100
    tables = ref.synthetic_tables(gen, (heads * groups, stages, 256, 8), (1.0, 0.5)[:stages], stage_axis=1)
    tables = tables + 1e-3 * torch.randn(tables.shape, generator=gen)
    codes = torch.randint(0, 256, (batch, heads, tokens, groups, stages), generator=gen, dtype=torch.uint8)
    given = tables.half() if tables_f16 else tables
    got = jkv.closed_loop_vq._ops.rvq_decode(codes.to(device), given.to(device), depth=depth, dtype=dtype)
    want = ref.frozen_decode(codes, tables, depth, dtype)
    assert torch.equal(got.cpu(), want)
