// Device weight-stream layout shared by the host packer and the HIP kernels.
//
// The weight of a layer is cut into items of 128 consecutive K-elements of one row:
// item (n, g) covers row n, elements [128g, 128g+128).  Items are stored in blocks of 64,
// one per lane of a wave64: block (t, sp) holds rows 16t..16t+15 times the four items
// 4sp..4sp+3 of each row ("span" sp = 512 K-elements), lane L = (n % 16) + 16 * (g % 4),
// which is the lane that feeds that row / K-quarter into a 16x16x32 MFMA.  Blocks are
// ordered t-major: block index = t * GS + sp with GS = ceil(K/512) spans per row; rows
// are padded to a multiple of 16 and the last span with zero bytes.  Inside a block
// every 16-byte chunk kind is contiguous over the 64 lanes, so one global_load_dwordx4
// of a wave reads 1 KiB of consecutive bytes.
//
//  GF4 block (6144 B):  chunk c = 0..3 at c*1024 + lane*16  -> 32 codes each
//                       chunk 4 at 4096 + lane*16           -> lo-byte tables A'|B'
//                       chunk 5 at 5120 + lane*16           -> hi-byte tables A'|B'
//  E2M1 block (4352 B): chunk c = 0..3 at c*1024 + lane*16  -> one 32-group each
//                       scales at 4096 + lane*4             -> E8M0 of groups 0..3
//
// GF4 nibble order inside each 32-bit word (8 elements e0..e7 of one item):
//   byte j (0..3) = code(e_j) | code(e_{j+4}) << 4
// so `w & 0x0F0F0F0F` yields the codes of e0..e3 and `(w >> 4) & 0x0F0F0F0F` those of
// e4..e7, one per byte, ready to be v_perm_b32 selectors.
// E2M1 words keep the canonical order (element 2j in the low nibble of byte j).
//
// GF4 codebook tables.  The 16 fp16 entries are split into a lo-byte plane T_lo[16]
// and a hi-byte plane T_hi[16]; each plane is stored as two 8-byte tables A', B' such
// that for every code c (selector byte s = c):
//     T[c] = perm8(A', s) ^ perm8(B', s ^ 8)
// where perm8 is the byte select of v_perm_b32: selectors 0..7 pick a table byte,
// 8..11 replicate the sign bit of table byte 1,3,5,7, 12 gives 0x00, 13..15 give 0xFF.
// A', B' are solved on the host (gf4_xor_tables) so the out-of-range half of each
// lookup cancels; the record is the same 32 bytes as the plain fp16 codebook.
#pragma once
#include <stdint.h>
#include <string.h>

namespace fb {

constexpr int kItemCodes = 128;   // K-elements per item
constexpr int kBlockItems = 64;   // items per block (one per lane)
constexpr int kGf4BlockBytes = 6144;
constexpr int kE2m1BlockBytes = 4352;

inline int block_bytes(int fmt) { return fmt == 0 ? kGf4BlockBytes : kE2m1BlockBytes; }

// Byte select of v_perm_b32 over an 8-byte table t[0..7] (t[0..3] = S1, t[4..7] = S0).
inline uint8_t perm8(const uint8_t* t, uint8_t sel) {
  if (sel >= 13) return 0xFF;
  if (sel == 12) return 0x00;
  if (sel >= 8) return (t[2 * (sel - 8) + 1] & 0x80) ? 0xFF : 0x00;
  return t[sel];
}

inline uint8_t rep(uint8_t b) { return (b & 0x80) ? 0xFF : 0x00; }

// Solves A', B' for one 16-entry byte plane T (see the header comment).
inline void gf4_xor_tables(const uint8_t T[16], uint8_t A[8], uint8_t B[8]) {
  A[4] = T[4];
  A[5] = T[5] ^ 0xFF;
  A[6] = T[6] ^ 0xFF;
  A[7] = T[7] ^ 0xFF;
  B[4] = T[12];
  B[5] = T[13] ^ 0xFF;
  B[6] = T[14] ^ 0xFF;
  B[7] = T[15] ^ 0xFF;
  A[3] = T[3] ^ rep(B[7]);
  A[2] = T[2] ^ rep(B[5]);
  B[3] = T[11] ^ rep(A[7]);
  B[2] = T[10] ^ rep(A[5]);
  A[1] = T[1] ^ rep(B[3]);
  B[1] = T[9] ^ rep(A[3]);
  A[0] = T[0] ^ rep(B[1]);
  B[0] = T[8] ^ rep(A[1]);
}

inline uint8_t gf4_lookup_plane(const uint8_t A[8], const uint8_t B[8], int c) {
  return (uint8_t)(perm8(A, (uint8_t)c) ^ perm8(B, (uint8_t)(c ^ 8)));
}

inline int64_t spans_per_row(int64_t K) { return (K / kItemCodes + 3) / 4; }
inline int64_t row_tiles(int64_t N) { return (N + 15) / 16; }
inline int64_t device_bytes(int64_t N, int64_t K, int fmt) {
  return row_tiles(N) * spans_per_row(K) * block_bytes(fmt);
}
// block offset and lane of item (n, g)
inline int64_t item_block(int64_t n, int64_t g, int64_t K) {
  return (n / 16) * spans_per_row(K) + g / 4;
}
inline int item_lane(int64_t n, int64_t g) { return (int)(n % 16 + 16 * (g % 4)); }

// Host: canonical 64 code bytes (128 codes) + 16 fp16 -> device item i.
inline void gf4_encode_item(const uint8_t* canon, const uint16_t* book, uint8_t* dev, int64_t n,
                            int64_t g, int64_t K) {
  uint8_t* base = dev + item_block(n, g, K) * kGf4BlockBytes;
  const int lane = item_lane(n, g);
  auto code = [&](int e) { return (uint8_t)((canon[e >> 1] >> ((e & 1) * 4)) & 15); };
  for (int c = 0; c < 4; ++c) {
    uint8_t* dst = base + c * 1024 + lane * 16;
    for (int d = 0; d < 4; ++d)
      for (int j = 0; j < 4; ++j) {
        const int e0 = c * 32 + d * 8 + j;
        dst[d * 4 + j] = (uint8_t)(code(e0) | (code(e0 + 4) << 4));
      }
  }
  uint8_t lo[16], hi[16];
  for (int t = 0; t < 16; ++t) {
    lo[t] = (uint8_t)(book[t] & 0xFF);
    hi[t] = (uint8_t)(book[t] >> 8);
  }
  uint8_t* tl = base + 4096 + lane * 16;
  uint8_t* th = base + 5120 + lane * 16;
  gf4_xor_tables(lo, tl, tl + 8);
  gf4_xor_tables(hi, th, th + 8);
}

// Host inverse of gf4_encode_item (decodes the tables through the perm8 model).
inline void gf4_decode_item(const uint8_t* dev, int64_t n, int64_t g, int64_t K, uint8_t* canon,
                            uint16_t* book) {
  const uint8_t* base = dev + item_block(n, g, K) * kGf4BlockBytes;
  const int lane = item_lane(n, g);
  memset(canon, 0, 64);
  for (int c = 0; c < 4; ++c) {
    const uint8_t* src = base + c * 1024 + lane * 16;
    for (int d = 0; d < 4; ++d)
      for (int j = 0; j < 4; ++j) {
        const int e0 = c * 32 + d * 8 + j;
        const uint8_t b = src[d * 4 + j];
        canon[e0 >> 1] |= (uint8_t)((b & 15) << ((e0 & 1) * 4));
        canon[(e0 + 4) >> 1] |= (uint8_t)((b >> 4) << (((e0 + 4) & 1) * 4));
      }
  }
  const uint8_t* tl = base + 4096 + lane * 16;
  const uint8_t* th = base + 5120 + lane * 16;
  for (int t = 0; t < 16; ++t)
    book[t] = (uint16_t)(gf4_lookup_plane(tl, tl + 8, t) | (gf4_lookup_plane(th, th + 8, t) << 8));
}

inline void e2m1_encode_item(const uint8_t* canon, const uint8_t* sc4, uint8_t* dev, int64_t n,
                             int64_t g, int64_t K) {
  uint8_t* base = dev + item_block(n, g, K) * kE2m1BlockBytes;
  const int lane = item_lane(n, g);
  for (int c = 0; c < 4; ++c) memcpy(base + c * 1024 + lane * 16, canon + c * 16, 16);
  memcpy(base + 4096 + lane * 4, sc4, 4);
}

inline void e2m1_decode_item(const uint8_t* dev, int64_t n, int64_t g, int64_t K, uint8_t* canon,
                             uint8_t* sc4) {
  const uint8_t* base = dev + item_block(n, g, K) * kE2m1BlockBytes;
  const int lane = item_lane(n, g);
  for (int c = 0; c < 4; ++c) memcpy(canon + c * 16, base + c * 1024 + lane * 16, 16);
  memcpy(sc4, base + 4096 + lane * 4, 4);
}

}  // namespace fb
