"""CPU models of LDS addressing in the GEMM kernels: the mid-size kernel's M/N-contiguous staging
(gemm_mid_kernel.hpp, gemm_tn_kernel.hpp) and the small-product kernel's int8 [k][row] staging
(gemm_generic.hip).

Each model restates the kernel's integer address arithmetic -- the LDS-DMA placement of a k-tile's
rows, the swizzle, and the addresses of the transposing fragment reads -- and checks what the
hardware contract requires of it: every byte of the slice is written exactly once by the DMA
instructions, every lane of every fragment receives the (k, column) element the MFMA operand map
expects (ds_read_b64_tr_b16 / ds_read_b64_tr_b8 semantics: in a 16-lane group, output lane i
element j comes from source lane 4 j + i / 4 (16-bit) or 2 j + i / 8 (8-bit)), every address stays
inside the 16 KB slice, and each 32-lane pass of a read touches all 64 banks exactly once whether
the hardware pairs lanes 0-31 / 32-63 or 16-lane groups {0, 2} / {1, 3}.  It also models the
unsigned-byte flip schedule: every fragment of every k-tile flipped once, after its read and before
its first MFMA, none past the last k-tile.  These pin the design's index algebra; the GPU tests
(test_gpu_gemm_mid.py, test_gpu_gemm_u8.py) pin the kernels themselves."""
from __future__ import annotations

import pytest

SLICE = 16 * 1024
PASSES = ([range(0, 32), range(32, 64)],
          [list(range(0, 16)) + list(range(32, 48)), list(range(16, 32)) + list(range(48, 64))])


def swz16(r):
    """TnSide<T, false, 128>::swz: 2 (r % 4) + 8 ((r / 8 + r / 16) % 2)."""
    return 2 * (r & 3) + 8 * (((r >> 3) ^ (r >> 4)) & 1)


def swz8(r):
    """TnSide<int8_t, false, 128>::swz: (r / 2 % 4) | 4 ((r / 16 + r / 32) % 2)."""
    return ((r >> 1) & 3) | ((((r >> 4) ^ (r >> 5)) & 1) << 2)


def banks_once(addrs, lanes):
    banks = []
    for lane in lanes:
        a = addrs[lane]
        banks += [(a // 4) % 64, (a // 4 + 1) % 64]   # 8 bytes per lane: two 4-byte banks
    return sorted(banks) == list(range(64))


def test_mn16_placement_reads_and_banks():
    """16-bit M/N-contiguous staging: 64 k rows x 256 bytes (128 columns)."""
    lds = {}
    for w in range(4):
        for i in range(4):
            for lane in range(64):
                rr, p = lane >> 4, lane & 15
                c = p ^ swz16(16 * w + 8 * (i >> 1) + rr)     # off[i / 2]
                krow = 16 * w + rr + 4 * i                     # row of off + i * step
                dst = w * 4096 + i * 1024 + 16 * lane          # LDS-DMA: lane l at dst + 16 l
                assert dst == krow * 256 + 16 * (c ^ swz16(krow))
                for e in range(8):
                    assert dst + 2 * e not in lds
                    lds[dst + 2 * e] = (krow, 8 * c + e)
    assert len(lds) == SLICE // 2
    for wx in range(2):
        for u in range(2):
            for t in range(4):
                lo, hi = {}, {}
                for lane in range(64):
                    ss, g = lane & 15, lane >> 4
                    f = swz16(8 * g + (ss >> 2))
                    b = u * 32 * 256 + (8 * g + (ss >> 2)) * 256 + 8 * (ss & 1) + ((8 * wx + 2 * t + ((ss & 3) >> 1)) ^ f) * 16
                    lo[lane], hi[lane] = b, b + 4 * 256
                    assert b + 4 * 256 + 8 <= SLICE
                for lane in range(64):
                    i, g = lane & 15, lane >> 4
                    for half, addrs in enumerate((lo, hi)):
                        for j in range(4):
                            krow, col = lds[addrs[16 * g + 4 * j + i // 4] + 2 * (i % 4)]
                            assert (krow, col) == (32 * u + 8 * g + 4 * half + j, 64 * wx + 16 * t + i)
                for addrs in (lo, hi):
                    for passes in PASSES:
                        for lanes in passes:
                            assert banks_once(addrs, lanes), (wx, u, t)


def test_mn8_placement_reads_and_banks():
    """8-bit M/N-contiguous staging: 128 k rows x 128 bytes (128 columns)."""
    lds = {}
    for w in range(4):
        for i in range(4):
            for lane in range(64):
                rr, p = lane >> 3, lane & 7
                c = p ^ swz8(32 * w + 16 * (i >> 1) + rr)
                krow = 32 * w + rr + 8 * i
                dst = w * 4096 + i * 1024 + 16 * lane
                assert dst == krow * 128 + 16 * (c ^ swz8(krow))
                for e in range(16):
                    assert dst + e not in lds
                    lds[dst + e] = (krow, 16 * c + e)
    assert len(lds) == SLICE
    for wx in range(2):
        for u in range(2):
            for t in range(4):
                lo, hi = {}, {}
                for lane in range(64):
                    s, g = lane & 15, lane >> 4
                    f = swz8(16 * g + (s >> 1))
                    b = u * 64 * 128 + (16 * g + (s >> 1)) * 128 + 8 * (s & 1) + ((4 * wx + t) ^ f) * 16
                    lo[lane], hi[lane] = b, b + 8 * 128
                    assert b + 8 * 128 + 8 <= SLICE
                for lane in range(64):
                    i, g = lane & 15, lane >> 4
                    for half, addrs in enumerate((lo, hi)):
                        for j in range(8):
                            krow, col = lds[addrs[16 * g + 2 * j + i // 8] + i % 8]
                            assert (krow, col) == (64 * u + 16 * g + 8 * half + j, 64 * wx + 16 * t + i)
                for addrs in (lo, hi):
                    for passes in PASSES:
                        for lanes in passes:
                            assert banks_once(addrs, lanes), (wx, u, t)


def test_swizzle_without_its_high_bit_conflicts():
    """The models can fail: dropping the (r / 8 + r / 16) term of the 16-bit swizzle leaves the two
    16-lane groups of a pass on the same chunk pairs."""
    def bad(r):
        return 2 * (r & 3)
    addrs = {}
    for lane in range(64):
        ss, g = lane & 15, lane >> 4
        addrs[lane] = (8 * g + (ss >> 2)) * 256 + 8 * (ss & 1) + ((2 * 0 + ((ss & 3) >> 1)) ^ bad(8 * g + (ss >> 2))) * 16
    assert not banks_once(addrs, range(0, 32))


def u8_schedule(ktiles):
    """gemm_mid_kernel's U8 flips: returns {(k-tile, k-step, fragment): flips}."""
    state, flips = {}, {}

    def rd(buf, tile, ks, t):
        state[(buf, t)] = [tile, ks, False]

    def flip(buf, t):
        st = state[(buf, t)]
        assert not st[2], ("flipped twice", buf, t, st)
        st[2] = True
        flips[(st[0], st[1], t)] = flips.get((st[0], st[1], t), 0) + 1

    def use(buf, q):   # MFMA q reads b[q % 4] (fragment 1 + q % 4) and a[q / 4] (0, or 4 + q / 4)
        for t in (1 + (q & 3), 0 if (q >> 2) == 0 else 4 + (q >> 2)):
            assert state[(buf, t)][2], ("used before its flip", buf, t, q)

    for t in range(8):
        rd("a", 0, 0, t)
    for t in range(8):
        flip("a", t)
    for kt in range(ktiles):
        for q in range(16):
            use("a", q)
            if q & 1:
                rd("b", kt, 1, q >> 1)
            if q in (2, 6) and kt > 0:
                flip("a", 6 + (q >> 2))
            if (q & 1) and q >= 5:
                flip("b", (q >> 1) - 2)
        for q in range(16):
            use("b", q)
            if not q & 1:
                rd("a", kt + 1, 0, q >> 1)
            if q in (2, 6):
                flip("b", 6 + (q >> 2))
            if not q & 1 and q >= 4 and kt + 1 < ktiles:
                flip("a", (q >> 1) - 2)
    return flips


@pytest.mark.parametrize("ktiles", [1, 2, 3, 8])
def test_u8_flip_schedule(ktiles):
    flips = u8_schedule(ktiles)
    assert flips == {(kt, ks, t): 1 for kt in range(ktiles) for ks in range(2) for t in range(8)}


def f8s(k):
    """gemm_small_kernel's int8 [k][row] swizzle: (k / 4 % 2) | 2 ((k / 16 + k / 32) % 2)."""
    return ((k >> 2) & 1) | ((((k >> 4) ^ (k >> 5)) & 1) << 1)


def small_i8_reads(f):
    """The small-product kernel's int8 [k][row] staging (512 k rows x 64 bytes, chunk j of k row k at
    slot j ^ f(k)) and its two ds_read_b64_tr_b8 per fragment; returns (lds map, per-read addresses)."""
    lds = {}
    for e in range(2048):                       # 16-byte chunk e of the K chunk: k row e / 4, column block e % 4
        k, j = e // 4, e % 4
        dst = k * 64 + 16 * (j ^ f(k))
        for b in range(16):
            assert dst + b not in lds
            lds[dst + b] = (k, 16 * j + b)
    reads = {}
    for ks in range(8):
        for rb in (0, 16, 32, 48):
            lo, hi = {}, {}
            for lane in range(64):
                g, s2 = lane >> 4, lane & 15
                k = ks * 64 + 16 * g + (s2 >> 1)
                p0 = k * 64 + 16 * ((rb >> 4) ^ f(k)) + 8 * (s2 & 1)
                lo[lane], hi[lane] = p0, p0 + 8 * 64
            reads[(ks, rb)] = (lo, hi)
    return lds, reads


def test_small_i8_placement_reads_and_banks():
    lds, reads = small_i8_reads(f8s)
    assert len(lds) == 512 * 64
    for (ks, rb), (lo, hi) in reads.items():
        for lane in range(64):
            i, g = lane & 15, lane >> 4
            for half, addrs in enumerate((lo, hi)):
                for j in range(8):      # tr8: output lane i byte j from source lane 2 j + i / 8, byte i % 8
                    k, col = lds[addrs[16 * g + 2 * j + i // 8] + i % 8]
                    assert (k, col) == (ks * 64 + 16 * g + 8 * half + j, rb + i)
        for addrs in (lo, hi):
            for passes in PASSES:
                for lanes in passes:
                    assert banks_once(addrs, lanes), (ks, rb)


def test_small_i8_swizzle_without_group_bit_conflicts():
    """Without its (k / 16 + k / 32) term the two 16-lane groups of a pass collide."""
    _, reads = small_i8_reads(lambda k: (k >> 2) & 1)
    lo, _ = reads[(0, 0)]
    assert not banks_once(lo, range(0, 32))
