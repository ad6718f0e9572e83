// LDS address maps of the MLP backward sweep's shared matrices and
// transposed-operand staging, and of the row-split Linear forward's 16-bit
// tile rows, as plain constexpr integer functions (no HIP types): the
// kernels build their lane addresses from these, and a host program compiled
// from this header alone enumerates the same addresses to check them against
// the LDS bank model below.
//
// LDS bank model of gfx950 (probed with per-lane address patterns and the
// SQ_LDS_BANK_CONFLICT counter; bank = dword address mod the bank count, no
// hashing of higher address bits; lanes of one pass that reach the same
// dword do not conflict; a pass takes as many cycles as the most distinct
// dwords any one bank serves):
//  - 2- and 4-byte reads and writes: lanes 0-31 and 32-63 in two passes over
//    32 banks;
//  - 8-byte reads: the same two passes over 64 banks;
//  - 16-byte reads: four passes of 16 lanes over 64 banks, each pass taking
//    two quads (4 lanes) of one 16-lane group and the other two quads of its
//    partner group: with q = (l >> 2) & 3 and group G = l >> 4, lane l is in
//    pass 2 (l >> 5) + (parity(q) ^ (G & 1)), i.e. lanes 0-3, 12-15, 20-27
//    form one pass and lanes 4-11, 16-19, 28-31 the next;
//  - 8-byte writes: four passes of 16 consecutive lanes over 32 banks;
//  - 16-byte writes: eight passes of 8 consecutive lanes over 32 banks.
//
// Offsets are in dwords (fp32 matrices) or in 8-byte slots (16-bit staging).
#pragma once

namespace ttt {
namespace lds {

// ---- fp32 matrix [rows][cols] as 16 x 16 blocks
// Block (R, C) starts at dword 256 (R cols/16 + C) = 16 R' cols + 16 C' for
// the block's first row R' = 16 R and column C' = 16 C, and element (r, c) of
// a block (r, c < 16) sits at
//     16 rowpos(r) + 4 ((c >> 2) ^ (r & 3)) + (c & 3),
// rowpos(r) taking the bits (r2, r0, r1, r3) of r as its bits 0..3: a row's
// 16-dword place has r2 in bit 0 (which 16-dword half of 32 banks), r0 in
// bit 1 (the quarter of 64 banks), and its four 4-dword chunks are permuted
// by r & 3.  The accesses and why none conflicts:
//  - C-layout tile (lane (g, n) at block row 4g + j, column n; 4-byte reads
//    and writes): the 32 lanes of a pass (g in {0, 1} or {2, 3}) have r2 = g &
//    1, i.e. opposite 16-dword halves, and within one g the chunk (n >> 2) ^ j
//    and n & 3 take all 16 places;
//  - row vector (lane (g, n) at block row n, columns 4g..4g+3; 16 bytes): a
//    read pass (quads n >> 2 in {0, 3} of one g, {1, 2} of g ^ 1) reaches
//    16 different (quarter, chunk) = ((n2, n0), g ^ (n & 3)) places of 64
//    banks, and a write pass (n = 0..7 or 8..15 of one g) 8 different
//    (half, chunk) = (n2, g ^ (n & 3)) places of 32 banks.
// Conflict-free 16-byte writes need rows n and n + 2 (and n + 1) in
// different places of 32 banks, so no two tile rows j of a lane lie a fixed
// distance apart: a view keeps one lane base per tile row.  No padding.
constexpr int rowpos(int r) { return ((r >> 2) & 1) | ((r & 1) << 1) | (((r >> 1) & 1) << 2) | (r & 8); }
constexpr int blk_elem(int r, int c) { return 16 * rowpos(r) + 4 * ((c >> 2) ^ (r & 3)) + (c & 3); }
// start of the block holding (r0, c0), both multiples of 16
constexpr int blk_base(int cols, int r0, int c0) { return r0 * cols + 16 * c0; }
// element (r, c) of the matrix
constexpr int mat_elem(int cols, int r, int c) { return blk_base(cols, r & ~15, c & ~15) + blk_elem(r & 15, c & 15); }
// lane (g, n)'s part of a tile access at block row 4g + j
constexpr int tile_lane(int g, int n, int j) { return blk_elem(4 * g + j, n); }
// lane (g, n)'s part of a row-vector access
constexpr int row_lane(int g, int n) { return blk_elem(n, 4 * g); }
// dword offset of a column offset cw (a multiple of 16) within block rows
constexpr int col_base(int cw) { return 16 * cw; }

// ---- 16-bit transposed operand frags of a [16 x 16 ft] matrix, written one
// element at a time by a [rows x features] owner and read as whole frags:
// frag lane L = 16 A + R of tile c (A = L >> 4) holds four 16-bit values in
// the 8-byte slot
//     66 c + 16 A + (R ^ 4A).
// The reads (slot per lane, 32-lane passes over 64 banks) reach 32 distinct
// slots mod 32 per pass.  The writes come from lane (lo, n) of wave w, row
// 4w + j, element n & 3 of frag lane 16 (n >> 2) + 4w + j of tile lo: slot
// 66 lo + 16 A + 4 (w ^ A) + j with A = n >> 2, so a pass (lo in {0, 1}, A in
// 0..3) covers 16 different dwords mod 32 (4 lo + 8 (w ^ A) + 2 j, and the
// half of the slot), two lanes writing the two halves of each.  The tile
// stride of 66 slots (not 64) is what separates lo = 0 and lo = 1.
constexpr int tfrag16_slot(int c, int lane) { return 66 * c + 16 * (lane >> 4) + ((lane & 15) ^ (4 * (lane >> 4))); }
// write side: slot of element (row 4w + j, feature n of tile lo), minus j
constexpr int tfrag16_put_slot(int lo, int w, int n) { return 66 * lo + 16 * (n >> 2) + 4 * (w ^ (n >> 2)); }
constexpr int tfrag16_bytes(int ft) { return 8 * (66 * (ft - 1) + 64); }

// ---- 16-bit C-layout tiles of a [16 x 16 ft] matrix gathered by rows: wave w
// writes the four rows 4w..4w+3 of feature l (lane l, tile lo = l >> 4, lane
// 16 w + n of it) as one 8-byte slot, and lane L of tile c reads its slot
//     64 c + (L ^ 16 (c & 1)).
// Both sides reach 32 distinct slots mod 32 in every 32-lane pass: the
// writes of lo = 0 and lo = 1 land in opposite 16-slot halves.
constexpr int crow16_slot(int c, int lane) { return 64 * c + (lane ^ (16 * (c & 1))); }

// ---- 16-bit 16 x 16 tiles written by rows and read back transposed
// (ds_read_b64_tr_b16: lane l supplies the address of row 4 (l >> 4) +
// ((l & 15) >> 2), 4-column group l & 3, and receives the tile's C-layout
// frag).  8-byte place of row m, group g:
//     4 m + (g ^ ((m >> 2) & 3)),
// so that the rows of one 16-lane write pass (m and m + 4 would share banks
// at 4 m + g) reach all 32 banks; each 32-lane read pass takes rows 0..7 or
// 8..15, a permutation of 32 consecutive places.  The G tiles, written by
// lane (g, n) at row (n & 7) + 8 w of tile 2p + (n >> 3), also flip bit 1 of
// the group on odd tiles, so that the two tiles of one write pass take the
// two halves of the banks.
constexpr int trow_put(int m, int g) { return 4 * m + (g ^ ((m >> 2) & 3)); }
constexpr int trow_get(int l) { return trow_put(4 * (l >> 4) + ((l & 15) >> 2), l & 3); }
constexpr int grow_put(int o, int t, int g) { return trow_put(t, g ^ (2 * (o & 1))); }
constexpr int grow_get(int o, int l) { return grow_put(o, 4 * (l >> 4) + ((l & 15) >> 2), l & 3); }

}  // namespace lds
}  // namespace ttt
