"""Host emulation of the skinny kernel's MFMA lane maps (no GPU).

In miori_amd/csrc/skinny.hip each lane (row n = lane % 16, quarter
c = lane / 16) loads 16 contiguous bytes of its weight row per K block; the
exact modes then exchange words between lane quarters with
v_permlane32_swap / v_permlane16_swap so that each 32-k MFMA step stays inside
one quantisation group, and the x fragments are loaded at `kmap(c, r)`. An
MFMA step multiplies, per quarter, the 8 weights of the lane's B fragment with
the 8 x values of the matching A fragment, so the kernel is right only if,
for every step r and quarter c:
  * the k of the B fragment's 8 elements (after the swaps and the unpacking
    order) equal, element by element, the k of the A fragment's 8 elements
    (x loaded at kmap(c, r), then pair-permuted by x_frag);
  * in the exact modes, all 32 k of the step lie in one group of size G.
The formulas below restate the kernel's load offsets, swap semantics, nibble
and byte unpacking orders, x_frag and kmap; a change to one of them that
breaks the pairing fails here before any GPU run."""
import numpy as np
import pytest

Q4X, Q8X, Q4F = 0, 1, 2


def kmap(mode, G, c, r):
    """skinny.hip kmap<MODE, G>(c, r): k offset (in the block) of the 8 x
    values quarter c supplies in step r."""
    if mode == Q4X and G == 32:
        return 32 * r + 8 * c
    if mode == Q4X and G == 64:
        return 32 * ((c & 1) + 2 * (r >> 1)) + 8 * ((r & 1) + 2 * (c >> 1))
    if mode == Q8X:
        return 32 * r + 8 * (((c & 1) << 1) | (c >> 1))
    return 32 * c + 8 * r


def permlane32_swap(a, b):
    """v_permlane32_swap a, b: lanes 32-63 of a trade places with lanes 0-31
    of b (the builtin returns the new a and b)."""
    a, b = a.copy(), b.copy()
    a_hi = a[32:].copy()
    a[32:] = b[:32]
    b[:32] = a_hi
    return a, b


def permlane16_swap(a, b):
    """v_permlane16_swap a, b: in each 32-lane half, lanes 16-31 of a trade
    places with lanes 0-15 of b."""
    a, b = a.copy(), b.copy()
    for base in (0, 32):
        hi = a[base + 16:base + 32].copy()
        a[base + 16:base + 32] = b[base:base + 16]
        b[base:base + 16] = hi
    return a, b


def loaded_words(mode, k0=0):
    """Per lane, the k of each element of its 4 loaded words: shape
    [64 lanes][4 words][elements per word] (4-bit: 8 nibbles in bit order,
    8-bit: 4 bytes)."""
    per = 8 if mode in (Q4X, Q4F) else 4
    w = np.zeros((64, 4, per), dtype=np.int64)
    for lane in range(64):
        c = lane >> 4
        # 4-bit: byte k0/2 + 16c of the row = k0 + 32c; 8-bit: k0 + 16c
        base = k0 + (32 * c if per == 8 else 16 * c)
        for t in range(4):
            w[lane, t] = base + per * t + np.arange(per)
    return w


def b_fragment_k(mode, G, r):
    """k of the 8 B-fragment elements of every lane in step r, in MFMA
    element order, following the kernel's swaps and unpacking."""
    w = loaded_words(mode)
    words = [w[:, t].copy() for t in range(4)]
    if mode == Q8X or (mode == Q4X and G in (32, 64)):
        words[0], words[2] = permlane32_swap(words[0], words[2])
        words[1], words[3] = permlane32_swap(words[1], words[3])
    if mode == Q4X and G == 32:
        words[0], words[1] = permlane16_swap(words[0], words[1])
        words[2], words[3] = permlane16_swap(words[2], words[3])
    out = np.zeros((64, 8), dtype=np.int64)
    if mode == Q4X:
        # nib2(v >> 4j): dword j = (nibble j, nibble j + 4) -> elements 2j, 2j+1
        v = words[r]
        for j in range(4):
            out[:, 2 * j] = v[:, j]
            out[:, 2 * j + 1] = v[:, j + 4]
    elif mode == Q8X:
        # codes8_bf16(wv[2r], wv[2r+1]): bytes of the first word then the second
        out[:, :4] = words[2 * r]
        out[:, 4:] = words[2 * r + 1]
    else:
        # Q4F: lo = v & 0x0F0F0F0F, hi = (v >> 4) & 0x0F0F0F0F; dword q =
        # (byte q of lo, byte q of hi) = (nibble 2q, nibble 2q + 1)
        v = words[r]
        for q in range(4):
            out[:, 2 * q] = v[:, 2 * q]
            out[:, 2 * q + 1] = v[:, 2 * q + 1]
    return out


def a_fragment_k(mode, G, r):
    """k of the 8 A-fragment (x) elements of every lane in step r: the 8
    consecutive x at kmap(c, r), pair-permuted by x_frag for 4-bit exact."""
    out = np.zeros((64, 8), dtype=np.int64)
    for lane in range(64):
        base = kmap(mode, G, lane >> 4, r)
        x = base + np.arange(8)
        if mode == Q4X:
            x = np.array([x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]])
        out[lane] = x
    return out


CASES = [(Q4X, 32), (Q4X, 64), (Q4X, 128), (Q8X, 32), (Q8X, 64), (Q8X, 128), (Q4F, 64)]


@pytest.mark.parametrize("mode,G", CASES)
def test_fragments_pair_up(mode, G):
    steps = 2 if mode == Q8X else 4   # 64-k blocks (8-bit) or 128-k blocks
    kb = 32 * steps
    seen = []
    for r in range(steps):
        b = b_fragment_k(mode, G, r)
        a = a_fragment_k(mode, G, r)
        assert np.array_equal(a, b), f"step {r}: x and weight k differ"
        ks = b.reshape(-1)
        seen.append(np.unique(ks))
        if mode in (Q4X, Q8X):
            for c in range(4):
                grp = set((b[16 * c:16 * c + 16] // G).reshape(-1).tolist())
                assert len(grp) == 1
            assert len(set((ks // min(G, kb)).tolist())) == 1, f"step {r} spans groups"
    # every k of the block is used exactly once per row over the steps
    allk = np.concatenate(seen)
    assert sorted(allk.tolist()) == list(range(kb))


def test_swaps_are_involutions():
    rng = np.random.default_rng(0)
    a, b = rng.integers(0, 1 << 30, 64), rng.integers(0, 1 << 30, 64)
    for f in (permlane32_swap, permlane16_swap):
        a2, b2 = f(*f(a, b))
        assert np.array_equal(a2, a) and np.array_equal(b2, b)


def test_map_catches_a_wrong_kmap():
    """The check is not vacuous: the 4-bit G=64 kmap without its quarter
    exchange term pairs x with the wrong weights."""
    b = b_fragment_k(Q4X, 64, 0)
    a = np.zeros_like(b)
    for lane in range(64):
        base = 32 * (lane >> 4)  # the no-exchange map
        x = base + np.arange(8)
        a[lane] = [x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]]
    assert not np.array_equal(a, b)
