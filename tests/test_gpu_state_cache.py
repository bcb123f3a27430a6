"""GPU tests of the slot-indexed decode step and the decode state cache.

``vmi_sssd_step_slots`` runs the same per-head arithmetic as the dense step, so every
check here is exact equality against the dense kernels run on explicit copies of the
states (which are themselves pinned to the oracle by test_gpu_sssd.py): the cache must
give each branch exactly the state an independent copy would have, as the reference's
copied ``layer_states`` lists do (``acd_engine.py:85-92``, ``hyper_generate.py:97-121``).
"""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _tokens(B, H, D, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, 1, H, D, generator=g), dim=-1).to(dtype)
    k = F.normalize(torch.randn(B, 1, H, D, generator=g), dim=-1).to(dtype)
    v = F.normalize(torch.randn(B, 1, H, D, generator=g), dim=-1).to(dtype)
    d = (0.5 * torch.sigmoid(torch.randn(B, 1, H, generator=g))).to(dtype)
    return q, k, v, d


def _orth(n, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.linalg.qr(torch.randn(n, H, D, D, generator=g))[0].contiguous()


def _step_slots(pool, q, k, v, d, src, dst):
    from verace_amd import _lib
    lib = _lib.load()
    B, _, H, D = q.shape
    out = torch.empty_like(q)
    s_dev = torch.tensor(src, dtype=torch.int32, device=pool.device)
    d_dev = torch.tensor(dst, dtype=torch.int32, device=pool.device)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    _lib.check(lib.vmi_sssd_step_slots(P(q), P(k), P(v), P(d), _lib.dtype_code(q.dtype),
                                       _lib.dtype_code(d.dtype), P(pool), pool.shape[0], P(s_dev),
                                       P(d_dev), P(out), B, H, D,
                                       _lib.stream_handle(pool.device)), "step_slots")
    return out


@pytest.mark.parametrize("D,dtype", [(128, torch.bfloat16), (128, torch.float32), (64, torch.bfloat16)])
def test_step_slots_equals_dense_step(device, D, dtype):
    from verace_amd import sssd_step_
    print(f"[case] step_slots D={D} {dtype}", flush=True)
    N, B, H = 20, 12, 8
    pool0 = _orth(N, H, D, seed=1)
    # in place, out of place into free slots, identity starts, an out-of-range input
    # (reads as the identity) and an out-of-range output (state write dropped)
    src = [3, 4, 5, -1, 7, 8, -1, 10, 11, 12, 25, 14]
    dst = [3, 0, 5, 1, 7, 2, 6, 10, 15, 12, 9, -1]
    q, k, v, d = (t.to(device) for t in _tokens(B, H, D, seed=D, dtype=dtype))
    pool = pool0.to(device)
    out = _step_slots(pool, q, k, v, d, src, dst)
    eye = torch.eye(D).expand(H, D, D)
    dense = torch.stack([pool0[s] if 0 <= s < N else eye for s in src]).contiguous().to(device)
    out_ref = sssd_step_(q, k, v, d, dense)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out_ref.cpu())
    pool = pool.cpu()
    dense = dense.cpu()
    written = set()
    for b, s in enumerate(dst):
        if 0 <= s < N:
            assert torch.equal(pool[s], dense[b]), b
            written.add(s)
    for s in range(N):
        if s not in written:
            assert torch.equal(pool[s], pool0[s]), s


def test_cache_tree_search_matches_independent_copies(device):
    """Prefill states written to the cache, each sequence forked into branches, branches
    stepped over two layers, a winner adopted and the rest released, then more steps:
    every output and state equals the dense step run on private copies."""
    from verace_amd import SSSDStateCache, sssd_step_
    print("[case] cache tree search", flush=True)
    L, H, D, nseq, nbr = 2, 8, 128, 3, 4
    cache = SSSDStateCache(L, 32, H, D, device=device)
    seqs = cache.new(nseq)
    ref = {}   # handle -> list of per-layer dense states (private copies)
    for l in range(L):
        st = _orth(nseq, H, D, seed=10 + l).to(device)
        cache.write(l, seqs, st)
        for i, h in enumerate(seqs):
            ref.setdefault(h, [None] * L)[l] = st[i:i + 1].clone()
    branches = []
    for h in seqs:
        for c in cache.fork(h, nbr):
            ref[c] = [x.clone() for x in ref[h]]
            branches.append(c)

    def step_all(handles, seed):
        for l in range(L):
            q, k, v, d = (t.to(device) for t in _tokens(len(handles), H, D, seed=seed + l))
            o = cache.step(l, q, k, v, d, handles)
            for b, h in enumerate(handles):
                o_ref = sssd_step_(q[b:b + 1], k[b:b + 1], v[b:b + 1], d[b:b + 1], ref[h][l])
                assert torch.equal(o[b:b + 1], o_ref), (h, l)

    step_all(branches, seed=100)
    # the parents were never stepped: their cached states are untouched
    for l in range(L):
        got = cache.read(l, seqs)
        for i, h in enumerate(seqs):
            assert torch.equal(got[i:i + 1], ref[h][l])
    # adopt branch 1 of every sequence, drop the rest and the parents
    winners = [branches[i * nbr + 1] for i in range(nseq)]
    cache.release([h for h in branches if h not in winners] + seqs)
    step_all(winners, seed=200)
    step_all(winners, seed=300)
    for l in range(L):
        got = cache.read(l, winners)
        for i, h in enumerate(winners):
            assert torch.equal(got[i:i + 1], ref[h][l])
        # only the winners' slots are held now
        assert cache.table.free_slots(l) == 32 - nseq


def test_forward_cached_matches_forward(device):
    """Module level: a prefill then single-token steps through the cache equal the
    reference-style forward with initial_state / return_state threading."""
    from verace_amd import SSSDAttention, SSSDStateCache
    print("[case] forward_cached", flush=True)
    torch.manual_seed(0)
    hidden, H, D, B = 256, 2, 128, 3
    m = SSSDAttention(hidden, H, D).to(device).to(torch.bfloat16)
    cache = SSSDStateCache(1, 8, H, D, device=device)
    hs = cache.new(B)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, 40, hidden, generator=g).to(torch.bfloat16).to(device)
    with torch.no_grad():
        y_ref, st = m(x, return_state=True)
        y = m.forward_cached(x, cache, 0, hs)
        assert torch.allclose(y.float(), y_ref.float(), rtol=0, atol=1e-6)
        for t in range(3):
            xt = torch.randn(B, 1, hidden, generator=g).to(torch.bfloat16).to(device)
            y_ref, st = m(xt, initial_state=st, return_state=True)
            y = m.forward_cached(xt, cache, 0, hs)
            assert torch.allclose(y.float(), y_ref.float(), rtol=0, atol=1e-6), t
        assert torch.allclose(cache.read(0, hs), st, rtol=0, atol=1e-6)


@pytest.mark.parametrize("D", [128, 64])
def test_cache_step_batch_above_one_launch(device, D):
    """300 handles (two launches of at most 256 items), half of them forked from the
    other half, against the dense step on copies."""
    from verace_amd import SSSDStateCache, sssd_step_
    print(f"[case] cache 300 handles D={D}", flush=True)
    H = 2
    cache = SSSDStateCache(1, 500, H, D, device=device)   # 150 held + 300 fresh (copy-on-write)
    base = cache.new(150)
    st0 = _orth(150, H, D, seed=3).to(device)
    cache.write(0, base, st0)
    kids = [cache.fork(h, 1)[0] for h in base]
    hs = [x for pair in zip(base, kids) for x in pair]
    ref = torch.cat([st0, st0]).reshape(2, 150, H, D, D).transpose(0, 1).reshape(300, H, D, D).contiguous()
    q, k, v, d = (t.to(device) for t in _tokens(300, H, D, seed=9))
    o = cache.step(0, q, k, v, d, hs)
    o_ref = sssd_step_(q, k, v, d, ref)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)
    assert torch.equal(cache.read(0, hs), ref)
    assert cache.table.free_slots(0) == 500 - 300   # the 150 shared slots were freed


def test_cache_tree_search_against_oracle_with_holograms(device):
    """Each tree-search branch (hyper_generate.py:97-121) against the oracle run from its
    parent's state: a 2-layer cache holding both halves of the reference's per-layer tuple
    (sssd_state [H, D, D] and the CHAM hologram, acd_engine.py:88-92).  Sequences are
    prefilled (states written), forked into branches that share the parent's slots, and every
    branch takes its own tokens for two steps (SSSD step, then the CHAM step of the same layer
    and handles).  Each branch's outputs and final states must equal the fp64 closed-form SSSD
    scan (oracle.sssd_closed) and the fp64 CHAM closed form (oracle.cham_scan) run from the
    parent's state over that branch's tokens, and the parents' own states must be untouched.
    Bars: bf16 I/O 2e-2 (outputs), fp32 states 1e-5."""
    from oracle import cham_scan, sssd_closed
    from verace_amd import SSSDStateCache
    print("[case] cache tree search vs oracle, with holograms", flush=True)
    L, N, H, D, h = 2, 64, 4, 128, 64
    n_seq, n_br, steps = 3, 3, 2
    cache = SSSDStateCache(L, N, H, D, device=device, hologram_dim=h)
    g = torch.Generator().manual_seed(40)
    parents = cache.new(n_seq)
    psi0 = {l: _orth(n_seq, H, D, seed=50 + l) for l in range(L)}
    holo0 = {}
    for l in range(L):
        a = torch.randn(n_seq, h, h, generator=g, dtype=torch.float64) + \
            1j * torch.randn(n_seq, h, h, generator=g, dtype=torch.float64)
        u = torch.linalg.qr(a)[0]
        holo0[l] = (u.real.float().contiguous(), u.imag.float().contiguous())
        cache.write(l, parents, psi0[l].to(device), (holo0[l][0].to(device), holo0[l][1].to(device)))
    branches = {p: cache.fork(p, n_br) for p in parents}
    order = [b for p in parents for b in branches[p]]
    nb = len(order)
    # per-branch tokens for every step and layer
    toks = {}
    for s in range(steps):
        for l in range(L):
            q, k, v, d = _tokens(nb, H, D, seed=1000 + 10 * s + l)
            cq = F.normalize(torch.randn(nb, 1, h, generator=g), dim=-1).bfloat16()
            ck = F.normalize(torch.randn(nb, 1, h, generator=g), dim=-1).bfloat16()
            cv = F.normalize(torch.randn(nb, 1, h, generator=g), dim=-1).bfloat16()
            cg = (0.1 * torch.sigmoid(torch.randn(nb, generator=g))).bfloat16()
            toks[(s, l)] = (q, k, v, d, cq, ck, cv, cg)
    outs = {}
    hs = np.array(order, dtype=np.int64)
    for s in range(steps):
        for l in range(L):
            q, k, v, d, cq, ck, cv, cg = (t.to(device) for t in toks[(s, l)])
            o = cache.step(l, q, k, v, d, hs)
            co = cache.cham_step(l, cq, ck, cv, cg, hs)
            outs[(s, l)] = (o.float().cpu(), co.float().cpu())
    torch.cuda.synchronize()
    worst = {"o": 0.0, "psi": 0.0, "co": 0.0, "holo": 0.0}

    def rel(a, b):
        a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
        return float(np.linalg.norm(a - b) / np.linalg.norm(b))
    for l in range(L):
        st = cache.read(l, order).cpu()
        hr, hi = (t.cpu() for t in cache.read_holograms(l, order))
        for i, bh in enumerate(order):
            pi = parents.index(next(p for p in parents if bh in branches[p]))
            sel = lambda t: torch.stack([toks[(s, l)][t][i] for s in range(steps)], 0).unsqueeze(0)
            q, k, v, d = (sel(j).float().numpy().reshape(1, steps, H, -1) if j < 3 else
                          sel(j).float().numpy().reshape(1, steps, H) for j in range(4))
            o64, p64 = sssd_closed.sssd_scan_closed_np(q, k, v, d, psi0[l][pi:pi + 1].double().numpy())
            got_o = torch.stack([outs[(s, l)][0][i, 0] for s in range(steps)], 0).numpy()
            worst["o"] = max(worst["o"], rel(got_o, o64[0]))
            worst["psi"] = max(worst["psi"], rel(st[i].numpy(), p64[0]))
            cq, ck, cv = (torch.stack([toks[(s, l)][4 + j][i, 0] for s in range(steps)], 0)
                          .double().numpy()[None] for j in range(3))
            cg = np.array([[float(toks[(s, l)][7][i]) for s in range(steps)]])
            rec, (sr, si) = cham_scan.cham_scan_closed(cq, ck, cv, cg, holo0[l][0][pi:pi + 1].double().numpy(),
                                                      holo0[l][1][pi:pi + 1].double().numpy())
            got_c = torch.stack([outs[(s, l)][1][i, 0] for s in range(steps)], 0).numpy()
            worst["co"] = max(worst["co"], rel(got_c, rec[0]))
            worst["holo"] = max(worst["holo"], rel(hr[i].numpy(), sr[0]), rel(hi[i].numpy(), si[0]))
        # the parents' states are untouched (their branches wrote fresh slots)
        assert torch.equal(cache.read(l, parents).cpu(), psi0[l])
        pr, pim = (t.cpu() for t in cache.read_holograms(l, parents))
        assert torch.equal(pr, holo0[l][0]) and torch.equal(pim, holo0[l][1])
    print("  " + " ".join(f"{k}={v:.2e}" for k, v in worst.items()), flush=True)
    assert worst["o"] <= 2e-2 and worst["co"] <= 2e-2
    assert worst["psi"] <= 1e-5 and worst["holo"] <= 1e-5
    # a CHAM step whose handles differ from the layer's last SSSD step is refused
    with pytest.raises(ValueError):
        q, k, v, d, cq, ck, cv, cg = (t.to(device) for t in toks[(0, 0)])
        cache.step(0, q, k, v, d, hs)
        cache.cham_step(0, cq[:2], ck[:2], cv[:2], cg[:2], hs[:2])


def test_cham_step_decisions_are_spent_once(device):
    """vmi_state_cache_cham_step replays the slot decisions of the layer's last SSSD step: only
    once, and not after a fork, a release or another plan of the layer (each can free or share
    the recorded slots, so a replay would copy into a slot that is now in place or reused)."""
    from verace_amd import SSSDStateCache
    print("[case] cham_step decisions are spent once", flush=True)
    H, D, h = 2, 128, 64
    cache = SSSDStateCache(2, 16, H, D, device=device, hologram_dim=h)
    g = torch.Generator().manual_seed(3)

    def cham_tok(n):
        return (F.normalize(torch.randn(n, 1, h, generator=g), dim=-1).bfloat16().to(device),
                F.normalize(torch.randn(n, 1, h, generator=g), dim=-1).bfloat16().to(device),
                F.normalize(torch.randn(n, 1, h, generator=g), dim=-1).bfloat16().to(device),
                (0.1 * torch.sigmoid(torch.randn(n, generator=g))).bfloat16().to(device))
    hs = cache.new(2)

    def sssd_step():
        q, k, v, d = (t.to(device) for t in _tokens(2, H, D, seed=int(torch.randint(1 << 20, (1,), generator=g))))
        cache.step(0, q, k, v, d, hs)
    sssd_step()
    cache.cham_step(0, *cham_tok(2), hs)
    with pytest.raises(ValueError):            # the same step's decisions a second time
        cache.cham_step(0, *cham_tok(2), hs)
    sssd_step()
    (child,) = cache.fork(hs[0], 1)
    with pytest.raises(ValueError):            # a fork in between
        cache.cham_step(0, *cham_tok(2), hs)
    sssd_step()
    cache.release([child])
    with pytest.raises(ValueError):            # a release in between
        cache.cham_step(0, *cham_tok(2), hs)
    sssd_step()
    cache.table.plan_step(0, hs)
    with pytest.raises(ValueError):            # another plan of the layer in between
        cache.cham_step(0, *cham_tok(2), hs)
    # a plan of another layer leaves layer 0's decisions standing
    sssd_step()
    cache.table.plan_step(1, hs)
    cache.cham_step(0, *cham_tok(2), hs)
    torch.cuda.synchronize()
