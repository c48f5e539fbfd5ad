"""CPU model of the wgrad kernel's fp32 epilogue staging for 384-wide tiles (the kOutF32 /
kOutF32Acc branch of vark_body in ggemm-asm_amd/csrc/vark_kernel.h; no kernel launches).

Each m-block of a wave's 96 x 96 fp32 results goes through a 6 KiB LDS region: lane (s16, q) writes
row s16, 16-byte chunk 4j + q (j = 0..5), chunk c of row r stored at c ^ ((r >> 1) & 7); the read
back gives lane l row (l >> 3) + 8h, chunk (l & 7) + 8k (h = 0, 1; k = 0..2), whole 128-byte lines.
The model restates the kernel's address arithmetic (two write bases and two read bases per lane)
and checks: the bases equal the swizzle formula; every (row, chunk) is written once and read once;
the 16 lanes the LDS serves together touch 16 distinct 4-bank groups, on writes and on reads; each
read instruction covers 8 rows x 128 contiguous bytes.
"""
PITCH = 384   # bytes per staged row: 96 floats


def _phys(r, c):
    return r * PITCH + 16 * (c ^ ((r >> 1) & 7))


def _write_addr(s16, q, j):
    u = (s16 >> 1) & 7
    ub = (u >> 2) & 1
    wb = s16 * PITCH + 16 * (q ^ (u & 3))
    return (wb - 64 * ub if j & 1 else wb + 64 * ub) + 64 * j


def _read_addr(lane, h, k):
    r0 = lane >> 3
    ew = (lane & 7) ^ (r0 >> 1)
    rd0 = r0 * PITCH + 16 * ew
    rd1 = rd0 + 8 * PITCH + (-64 if ew & 4 else 64)
    return (rd1 if h else rd0) + 128 * k


def test_bases_follow_the_swizzle():
    for s16 in range(16):
        for q in range(4):
            for j in range(6):
                assert _write_addr(s16, q, j) == _phys(s16, 4 * j + q)
    for lane in range(64):
        for h in range(2):
            for k in range(3):
                assert _read_addr(lane, h, k) == _phys((lane >> 3) + 8 * h, 8 * k + (lane & 7))


def test_each_chunk_written_and_read_once():
    w = sorted(_write_addr(s, q, j) for s in range(16) for q in range(4) for j in range(6))
    r = sorted(_read_addr(l, h, k) for l in range(64) for h in range(2) for k in range(3))
    assert w == r == sorted(set(w)) and len(w) == 16 * 24
    assert max(w) + 16 <= 16 * PITCH <= 9216          # inside the wave's staging region


def test_bank_groups_conflict_free():
    group = lambda a: (a // 16) % 16                    # 16-byte group of 4 of the 64 banks
    for j in range(6):
        for q in range(4):                              # lanes 16q .. 16q + 15: s16 = 0..15
            assert len({group(_write_addr(s, q, j)) for s in range(16)}) == 16
    for h in range(2):
        for k in range(3):
            for g in range(4):
                assert len({group(_read_addr(l, h, k)) for l in range(16 * g, 16 * g + 16)}) == 16


def test_reads_are_whole_lines():
    for h in range(2):
        for k in range(3):
            rows = {}
            for lane in range(64):
                r, c = (lane >> 3) + 8 * h, 8 * k + (lane & 7)
                rows.setdefault(r, []).append(c)
            assert len(rows) == 8
            for cs in rows.values():                     # 8 consecutive 16-byte chunks = 128 bytes
                assert sorted(cs) == list(range(8 * k, 8 * k + 8))
