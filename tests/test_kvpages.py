"""Paged KV bookkeeping (si_kv_pages_*, libsi_host.so) on the CPU: pages
handed out lowest id first, a sequence's table grows page by page, freed
pages are reused, exhaustion takes nothing, and a random workload keeps
every page owned by at most one sequence (checked against a Python model of
the same rules).  No counterpart in the reference (one contiguous cache per
layer, qwen_one_layer.c:262-266)."""
import numpy as np
import pytest

import si_amd


@pytest.fixture
def H():
    return si_amd.host_lib()


def _table(H, p, max_seqs, max_pages):
    t = H.si_kv_page_table(p)
    return np.ctypeslib.as_array(t, shape=(max_seqs * max_pages,)).reshape(max_seqs, max_pages)


def test_growth_reuse_and_exhaustion(H):
    p = H.si_kv_pages_create(6, 16, 3, 4)
    try:
        a, b = H.si_kv_seq_add(p), H.si_kv_seq_add(p)
        assert (a, b) == (0, 1)
        assert H.si_kv_seq_grow(p, a, 1) == 0 and H.si_kv_seq_len(p, a) == 1
        assert H.si_kv_seq_grow(p, a, 16) == 0  # still one page
        assert H.si_kv_pages_free(p) == 5
        assert H.si_kv_seq_grow(p, b, 40) == 0  # three pages
        assert H.si_kv_seq_grow(p, a, 17) == 0  # second page
        t = _table(H, p, 3, 4)
        assert list(t[a, :2]) == [0, 4] and list(t[b, :3]) == [1, 2, 3]
        assert H.si_kv_pages_free(p) == 1
        assert H.si_kv_seq_grow(p, b, 64) == 0  # the last free page
        assert H.si_kv_pages_free(p) == 0 and _table(H, p, 3, 4)[b, 3] == 5
        # exhaustion: nothing is taken and the length stays
        assert H.si_kv_seq_grow(p, a, 33) == -1
        assert H.si_kv_seq_len(p, a) == 17 and list(_table(H, p, 3, 4)[a]) == [0, 4, 0, 0]
        # beyond max_pages
        c = H.si_kv_seq_add(p)
        assert c == 2 and H.si_kv_seq_add(p) == -1
        assert H.si_kv_seq_grow(p, c, 65) == -1
        # free b: its pages return and are handed out again in order
        before = list(_table(H, p, 3, 4)[b])
        H.si_kv_seq_free(p, b)
        assert H.si_kv_pages_free(p) == 4
        assert list(_table(H, p, 3, 4)[b]) == [0, 0, 0, 0]
        d = H.si_kv_seq_add(p)
        assert d == b and H.si_kv_seq_grow(p, d, 64) == 0
        assert list(_table(H, p, 3, 4)[d]) == before
    finally:
        H.si_kv_pages_destroy(p)


def test_random_workload_matches_model(H):
    npages, ps, max_seqs, max_pages = 40, 8, 6, 12
    p = H.si_kv_pages_create(npages, ps, max_seqs, max_pages)
    rng = np.random.default_rng(0)
    free = list(range(npages - 1, -1, -1))  # stack, lowest id on top
    seqs = {}
    try:
        for step in range(3000):
            op = rng.integers(0, 10)
            if op == 0 and len(seqs) < max_seqs:
                sid = H.si_kv_seq_add(p)
                assert sid == min(set(range(max_seqs)) - set(seqs))
                seqs[sid] = [0, []]
            elif op == 1 and seqs:
                sid = int(rng.choice(list(seqs)))
                H.si_kv_seq_free(p, sid)
                free.extend(reversed(seqs.pop(sid)[1]))
            elif seqs:
                sid = int(rng.choice(list(seqs)))
                ln, pages = seqs[sid]
                new = ln + int(rng.integers(0, 20))
                need = -(-new // ps)
                ok = need <= max_pages and need - len(pages) <= len(free)
                assert H.si_kv_seq_grow(p, sid, new) == (0 if ok else -1)
                if ok:
                    while len(pages) < need:
                        pages.append(free.pop())
                    seqs[sid][0] = new
            t = _table(H, p, max_seqs, max_pages)
            held = []
            for sid, (ln, pages) in seqs.items():
                assert H.si_kv_seq_len(p, sid) == ln
                assert list(t[sid, :len(pages)]) == pages
                held += pages
            assert len(held) == len(set(held))  # no page owned twice
            assert H.si_kv_pages_free(p) == len(free) == npages - len(held)
    finally:
        H.si_kv_pages_destroy(p)
