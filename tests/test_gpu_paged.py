"""Paged KV cache and the multi-layer decode stack on the GPU (no
counterpart in the reference; the layer math is the reference's run_layer,
qwen_one_layer.c:237-281, checked with the chained oracle check):
  * si_attention_paged is bit-identical to si_attention on the same rows laid
    out contiguously (same kernels, same split), for shuffled page ids and
    page sizes 1, 16 and 64;
  * si_layer_decode_paged passes the chained layer check per sequence on
    the rows gathered back from the pool, and touches no other pool row;
  * the stack (si_stack_*, libsi_host.so) decoding sequences that join,
    grow across page boundaries and leave (their pages reused) gives the
    same bits as the same layers driven one by one from Python."""
import ctypes

import numpy as np
import pytest

import si_amd
from oracle.oracle_py import make_shape as or_shape
from tests.chain import E2E_BOUND, LayerBuffers, check_row, end_to_end_report
from tests.gpu_helpers import close, dev, device_view, empty, host, kv_history, make_layer

pytestmark = pytest.mark.gpu
_SHAPES = {
    "g1_d32": dict(hidden=256, qheads=8, kvheads=1, hdim=32, ffn=0),
    "0.5b": dict(si_amd.SHAPES["0.5b"], ffn=0),
    "g4_d96": dict(hidden=768, qheads=8, kvheads=4, hdim=96, ffn=0),
    "7b": dict(si_amd.SHAPES["7b"], ffn=0),
}


def _torch():
    import torch
    return torch


def _paged_layout(rng, ctxs, page_size, npages, max_pages):
    """Random distinct page ids for each sequence: table [nseq][max_pages]."""
    need = [-(-c // page_size) for c in ctxs]
    ids = rng.permutation(npages)[:sum(need)]
    table = np.zeros((len(ctxs), max_pages), np.int32)
    k = 0
    for i, n in enumerate(need):
        table[i, :n] = ids[k:k + n]
        k += n
    return table


def _to_pool(cache, ctxs, table, page_size, npages, kvd):
    """cache [nseq][max_ctx*kvd] -> pool [npages*page_size*kvd] (unused rows random)."""
    pool = np.random.default_rng(1).integers(0, 0x3c00, npages * page_size * kvd,
                                             dtype=np.uint16)
    for i, c in enumerate(ctxs):
        for p in range(c):
            r = table[i, p // page_size] * page_size + p % page_size
            pool[r * kvd:(r + 1) * kvd] = cache[i, p * kvd:(p + 1) * kvd]
    return pool


def _from_pool(pool, ctx, row_table, page_size, kvd):
    out = np.empty(ctx * kvd, np.uint16)
    for p in range(ctx):
        r = row_table[p // page_size] * page_size + p % page_size
        out[p * kvd:(p + 1) * kvd] = pool[r * kvd:(r + 1) * kvd]
    return out


@pytest.mark.parametrize("name", list(_SHAPES))
@pytest.mark.parametrize("page_size", [1, 16, 64])
def test_paged_attention_bit_identical(oracle, name, page_size):
    torch = _torch()
    sd = _SHAPES[name]
    s = si_amd.make_shape(**sd)
    kvd, QD = s.kvheads * s.hdim, s.qheads * s.hdim
    rng = np.random.default_rng(page_size + len(name))
    ctxs = [1, 5, 333, 64, 1000, 17, 128, 700]
    nq, max_ctx = len(ctxs), 1000
    max_pages = -(-max_ctx // page_size)
    npages = sum(-(-c // page_size) for c in ctxs) + 7
    print(f"paged attention {name} page {page_size}", flush=True)
    kc = np.stack([kv_history(oracle, rng, max_ctx, kvd) for _ in ctxs])
    vc = np.stack([kv_history(oracle, rng, max_ctx, kvd) for _ in ctxs])
    table = _paged_layout(rng, ctxs, page_size, npages, max_pages)
    kp = _to_pool(kc, ctxs, table, page_size, npages, kvd)
    vp = _to_pool(vc, ctxs, table, page_size, npages, kvd)
    q = dev(rng.standard_normal(nq * QD).astype(np.float32))
    ctx_dev = dev(np.array(ctxs, np.int32))
    wsb = si_amd.lib().si_attention_workspace(ctypes.byref(s), nq, max_ctx)
    ws = empty(wsb, torch.uint8)
    outs = []
    for paged in (False, True):
        attn = empty(nq * QD, torch.float32)
        qs = empty(nq * QD, torch.int8)
        d = empty(nq * QD // 32, torch.int16)
        if paged:
            kpd, vpd, td = dev(kp.view(np.int16)), dev(vp.view(np.int16)), dev(table)
            si_amd.call("si_attention_paged", ctypes.byref(s), si_amd.ptr(q), nq, si_amd.ptr(kpd),
                        si_amd.ptr(vpd), npages, page_size, si_amd.ptr(td), max_pages,
                        si_amd.ptr(ctx_dev), max_ctx, si_amd.ptr(attn), si_amd.ptr(qs),
                        si_amd.ptr(d), None, si_amd.ptr(ws), wsb, None)
        else:
            kcd, vcd = dev(kc.reshape(-1).view(np.int16)), dev(vc.reshape(-1).view(np.int16))
            si_amd.call("si_attention", ctypes.byref(s), si_amd.ptr(q), nq, si_amd.ptr(kcd),
                        si_amd.ptr(vcd), max_ctx * kvd, si_amd.ptr(ctx_dev), 0, 0, max_ctx,
                        si_amd.ptr(attn), si_amd.ptr(qs), si_amd.ptr(d), None, si_amd.ptr(ws),
                        wsb, None)
        torch.cuda.synchronize()
        outs.append((host(attn), host(qs), host(d)))
    for a, b in zip(*outs):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    # and the values are attention: sequence 2 against the oracle
    qh = host(q).reshape(nq, QD)
    want = oracle.attention_flash(or_shape(**sd), qh[2], kc[2], vc[2], ctxs[2])
    close(outs[1][0].reshape(nq, QD)[2], want, 2e-3, "paged vs oracle")


@pytest.mark.parametrize("flags", [si_amd.SI_LAYER_FULL, si_amd.SI_LAYER_EXACT,
                                   si_amd.SI_LAYER_ATTN_ONLY])
def test_layer_decode_paged_chain(oracle, flags):
    torch = _torch()
    full = not flags & si_amd.SI_LAYER_ATTN_ONLY
    sd = dict(si_amd.SHAPES["0.5b"])
    if not full:
        sd["ffn"] = 0
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    kvd = s.kvheads * s.hdim
    lay = make_layer(oracle, os_, 51, ffn=full)
    rng = np.random.default_rng(52)
    ctxs = [1, 40, 1024, 97, 300, 2]
    nseq, max_ctx, ps = len(ctxs), 1024, 32
    max_pages = max_ctx // ps
    npages = sum(-(-c // ps) for c in ctxs) + 3
    hist_k = np.stack([kv_history(oracle, rng, max_ctx, kvd) for _ in ctxs])
    hist_v = np.stack([kv_history(oracle, rng, max_ctx, kvd) for _ in ctxs])
    table = _paged_layout(rng, ctxs, ps, npages, max_pages)
    kp = _to_pool(hist_k, ctxs, table, ps, npages, kvd)
    vp = _to_pool(hist_v, ctxs, table, ps, npages, kvd)
    x = rng.standard_normal((nseq, s.hidden)).astype(np.float32)
    L = si_amd.Layer(s, lay, nseq, max_ctx)
    kpd, vpd = dev(kp.view(np.int16)), dev(vp.view(np.int16))
    out = empty(nseq * s.hidden, torch.float32)
    L.decode_paged(dev(x), nseq, kpd, vpd, npages, ps, dev(table), max_pages,
                   dev(np.array(ctxs, np.int32)), max_ctx, out, flags)
    torch.cuda.synchronize()
    B = LayerBuffers(L, os_, nseq)
    hk, hv = host(kpd).view(np.uint16), host(vpd).view(np.uint16)
    got = host(out).reshape(nseq, s.hidden)
    written = set()
    for i, c in enumerate(ctxs):
        kc_i = _from_pool(hk, c, table[i], ps, kvd)
        vc_i = _from_pool(hv, c, table[i], ps, kvd)
        # history rows unchanged
        assert np.array_equal(kc_i[:(c - 1) * kvd], hist_k[i, :(c - 1) * kvd])
        check_row(oracle, os_, lay, x[i], i, B, kc_i, vc_i, 0, c - 1, c, got[i],
                  bool(flags & si_amd.SI_LAYER_EXACT), full=full)
        written.add(table[i, (c - 1) // ps] * ps + (c - 1) % ps)
    # no other pool row was written
    rows = np.ones(npages * ps, bool)
    rows[list(written)] = False
    assert np.array_equal(hk.reshape(-1, kvd)[rows], kp.reshape(-1, kvd)[rows])
    assert np.array_equal(hv.reshape(-1, kvd)[rows], vp.reshape(-1, kvd)[rows])
    L.close()


def test_stack_matches_layers_driven_one_by_one(oracle):
    torch = _torch()
    H = si_amd.host_lib()
    sd = si_amd.SHAPES["0.5b"]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    kvd, nl, max_seqs, max_ctx, ps, npages = s.kvheads * s.hdim, 3, 4, 96, 16, 17
    lays = [make_layer(oracle, os_, 60 + l) for l in range(nl)]
    keep = [{k: np.ascontiguousarray(v) for k, v in t.items() if v is not None} for t in lays]
    hosts = (si_amd.LayerHost * nl)(*[si_amd.LayerHost(**{k: v.ctypes.data for k, v in kk.items()})
                                      for kk in keep])
    st = H.si_stack_create(ctypes.byref(s), ctypes.cast(hosts, ctypes.c_void_p), nl, max_seqs,
                           max_ctx, npages, ps)
    pages = H.si_stack_pages(st)
    max_pages = max_ctx // ps
    pool_elems = npages * ps * kvd
    mirror = [si_amd.Layer(s, lay, max_seqs, max_ctx) for lay in lays]
    mk = [torch.zeros(pool_elems, dtype=torch.int16, device="cuda") for _ in range(nl)]
    mv = [torch.zeros(pool_elems, dtype=torch.int16, device="cuda") for _ in range(nl)]
    # the stack's pools start uninitialised: the mirror starts from a copy
    for l in range(nl):
        for src, dst in ((H.si_stack_k_pool(st, l), mk[l]), (H.si_stack_v_pool(st, l), mv[l])):
            dst.copy_(device_view(src, pool_elems, torch.int16))
    rng = np.random.default_rng(61)
    active = []
    for step in range(40):
        if step in (0, 3, 9) and len(active) < max_seqs:
            active.append(H.si_kv_seq_add(pages))
        if step == 25:  # the second sequence leaves; a new one reuses its pages
            H.si_kv_seq_free(pages, active.pop(1))
            active.append(H.si_kv_seq_add(pages))
        ids = (ctypes.c_int * len(active))(*active)
        assert H.si_stack_prepare(st, ids, len(active)) == 0
        n = len(active)
        x = dev(rng.standard_normal((n, s.hidden)).astype(np.float32))
        out = empty(n * s.hidden, torch.float32)
        H.si_stack_decode(st, si_amd.ptr(x), si_amd.ptr(out), si_amd.SI_LAYER_FULL, None)
        # mirror: the same page lists and contexts, layer by layer
        tab = np.ctypeslib.as_array(H.si_kv_page_table(pages), shape=(max_seqs * max_pages,))
        tab = tab.reshape(max_seqs, max_pages)[active].astype(np.int32)
        ctx = np.array([H.si_kv_seq_len(pages, i) for i in active], np.int32)
        td, cd = dev(np.ascontiguousarray(tab)), dev(ctx)
        cur = x
        ins = []
        for l in range(nl):
            o = empty(n * s.hidden, torch.float32)
            ins.append(cur)
            mirror[l].decode_paged(cur, n, mk[l], mv[l], npages, ps, td, max_pages, cd,
                                   int(ctx.max()), o, si_amd.SI_LAYER_FULL)
            cur = o
        torch.cuda.synchronize()
        assert np.array_equal(host(out).view(np.uint32), host(cur).view(np.uint32)), step
        assert np.isfinite(host(out)).all()
        if step in (0, 39):
            # each layer of the last sequence against the oracle's layer on the
            # same input and the same cache rows gathered from the pool
            i, c = n - 1, int(ctx[n - 1])
            for l in range(nl):
                kc_i = _from_pool(host(mk[l]).view(np.uint16), c, tab[i], ps, kvd)
                vc_i = _from_pool(host(mv[l]).view(np.uint16), c, tab[i], ps, kvd)
                xin = host(ins[l]).reshape(n, s.hidden)[i]
                yout = host(ins[l + 1] if l + 1 < nl else cur).reshape(n, s.hidden)[i]
                want = oracle.layer_decode(os_, lays[l], xin, kc_i.copy(), vc_i.copy(), c)
                e2e = end_to_end_report(yout, want)
                assert e2e["max_over_rms"] <= E2E_BOUND["0.5b"], (step, l, e2e)
    for l in range(nl):
        assert torch.equal(device_view(H.si_stack_k_pool(st, l), pool_elems, torch.int16), mk[l])
        assert torch.equal(device_view(H.si_stack_v_pool(st, l), pool_elems, torch.int16), mv[l])
    # an exhausted pool is reported, nothing is taken
    big = H.si_kv_seq_len(pages, active[0])
    free_before = H.si_kv_pages_free(pages)
    assert H.si_kv_seq_grow(pages, active[0], max_ctx + 1) == -1
    assert H.si_kv_seq_len(pages, active[0]) == big
    assert H.si_kv_pages_free(pages) == free_before
    # exhaustion through si_stack_prepare: steps until the pool runs dry,
    # then the failed step leaves every length as it was and the stack
    # refuses to decode until a prepare succeeds
    assert H.si_stack_nseq(st) == len(active)
    active.append(H.si_kv_seq_add(pages))  # a fourth sequence: 17 pages run out first
    ids = (ctypes.c_int * len(active))(*active)
    while True:
        lens = [H.si_kv_seq_len(pages, a) for a in active]
        if max(lens) >= max_ctx:
            break
        if H.si_stack_prepare(st, ids, len(active)) != 0:
            assert [H.si_kv_seq_len(pages, a) for a in active] == lens
            assert H.si_kv_pages_free(pages) == 0
            assert H.si_stack_nseq(st) == 0
            break
    else:
        raise AssertionError("unreachable")
    assert H.si_stack_nseq(st) == 0, "the pool never ran dry"
    H.si_stack_destroy(st)
    for m in mirror:
        m.close()
