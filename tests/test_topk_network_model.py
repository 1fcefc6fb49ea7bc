"""A lane-level model of the MoE top-k merge network (kernels_amd/csrc/kq_moe_device.h:
topk_lists / topk_select), checked against repeated strict-greater argmax passes
(moe-fused/src/kernels.metal:149-156; oracle/kqref.c kqref_moe_router_f64), on the CPU.

The model follows the kernel step by step on 64 lanes: each lane sorts its own
candidate keys (2 columns, or 4 when experts 128-255 hold one), then six merges
of descending top-L lists -- DPP quad_perm [1,0,3,2] and [2,3,0,1], row_ror 4
and 8 inside each 16-lane row, then v_permlane16_swap and v_permlane32_swap of
each list register with itself -- each keeping max(a_i, b_{L-1-i}) and sorting
that bitonic list with a half-cleaner network. Pick j is the j-th key of the
merged list; its expert is the (o + 1)-th lowest index holding that key, o the
number of earlier picks with the same key. Keys are the kernel's
order-preserving integers (0: never selectable). The GPU tests run the kernel
itself (tests/test_gpu_moe.py: golden vector, ties, edge logits)."""
import numpy as np
import pytest

LANES = 64


def dpp(x, ctrl):
    i = np.arange(LANES)
    if ctrl == "xor1":
        src = (i & ~3) | np.array([1, 0, 3, 2])[i & 3]
    elif ctrl == "xor2":
        src = (i & ~3) | np.array([2, 3, 0, 1])[i & 3]
    elif ctrl == "ror4":
        src = (i & ~15) | ((i - 4) % 16)
    else:  # ror8
        src = (i & ~15) | ((i - 8) % 16)
    return x[src]


def bitonic_sort_desc(c):
    c = list(c)
    h = len(c) // 2
    while h >= 1:
        for i in range(len(c)):
            if i & h == 0:
                x, y = c[i], c[i + h]
                c[i], c[i + h] = np.maximum(x, y), np.minimum(x, y)
        h //= 2
    return c


def merge(a, partner):
    L = len(a)
    return bitonic_sort_desc([np.maximum(a[i], partner(a[L - 1 - i])) for i in range(L)])


def permlane_swap(x, halves):
    """v_permlane{32,16}_swap of a register with itself: (new vdst, new vsrc)."""
    if halves:
        return np.concatenate([x[:32], x[:32]]), np.concatenate([x[32:], x[32:]])
    r = x.reshape(4, 16)
    return np.concatenate([r[0], r[0], r[2], r[2]]), np.concatenate([r[1], r[1], r[3], r[3]])


def merge_swap(a, halves):
    L = len(a)
    lo, hi = zip(*[permlane_swap(a[i], halves) for i in range(L)])
    return bitonic_sort_desc([np.maximum(lo[i], hi[L - 1 - i]) for i in range(L)])


def network_topk(k, tk):
    """k: [4][64] candidate keys (expert lane + 64 c in column c)."""
    wide = bool(np.any(k[2] | k[3]))
    nc, L = (4 if wide else 2), (4 if tk <= 4 else 8)
    a = [np.zeros(LANES, np.uint64) for _ in range(L)]
    s = np.sort(np.stack(k[:nc]), axis=0)[::-1]
    for c in range(nc):
        a[c] = s[c].copy()
    for ctrl in ("xor1", "xor2", "ror4", "ror8"):
        a = merge(a, lambda v, ctrl=ctrl: dpp(v, ctrl))
    a = merge_swap(a, halves=False)
    a = merge_swap(a, halves=True)
    for i in range(L):  # every lane holds the same sorted list
        assert np.all(a[i] == a[i][0])
    picks, occ, prev = [], 0, 0
    for j in range(tk):
        r = int(a[j][0]) if j < L else 0
        occ = occ + 1 if j > 0 and r == prev else 0
        prev = r
        if r == 0:
            picks.append((0, 0))
            continue
        idx = sorted(64 * c + l for c in range(nc) for l in np.nonzero(k[c] == r)[0])
        picks.append((idx[occ], r))
    return picks


def argmax_passes(k, tk):
    keys = np.concatenate(k).astype(np.int64)
    out = []
    for _ in range(tk):
        bi, bv = 0, 0
        for e in range(keys.size):
            if keys[e] > bv:  # strict: the lowest index among equals
                bv, bi = keys[e], e
        out.append((bi, bv))
        if bv:
            keys[bi] = 0
    return out


@pytest.mark.parametrize("seed", range(6))
def test_network_matches_argmax_passes(seed):
    rng = np.random.default_rng(seed)
    for _ in range(300):
        ne = int(rng.choice([8, 16, 100, 128, 130, 200, 256]))
        tk = int(rng.integers(1, 9))
        nvals = int(rng.choice([2, 5, 50, 10 ** 6]))  # few values: many ties
        keys = rng.integers(1, nvals + 1, 256).astype(np.uint64)
        keys[rng.random(256) < rng.choice([0.0, 0.3, 0.97])] = 0  # NaN / -inf / removed
        keys[ne:] = 0  # past the last expert
        k = [keys[64 * c:64 * c + 64] for c in range(4)]
        assert network_topk(k, tk) == argmax_passes(k, tk), (ne, tk, nvals)


def test_ties_across_columns_take_the_lower_index():
    keys = np.zeros(256, np.uint64)
    keys[[7, 135, 64, 200]] = [9, 9, 8, 8]
    k = [keys[64 * c:64 * c + 64] for c in range(4)]
    assert [e for e, _ in network_topk(k, 4)] == [7, 135, 64, 200]
