#pragma once
// Device layout of quantized weights and activations, shared by the host (which repacks a weight on upload) and
// the kernels. Plain C++ (no HIP), so hip_backend.cpp includes it too.
//
// nibble's weights are ggml blocks (src/quant.h:34-110): 18, 22, 24, 34, 144, 176 or 210 bytes, so a block in a
// row starts at any even address and its fields are not aligned for vector loads. On upload each weight is split
// into planes, one per field, every plane 256-byte aligned and every block's part of it 4- or 16-byte aligned:
//   q  the quants: Q4_0 / Q5_0 / Q5_1 16 bytes (nibbles as stored), Q8_0 32, Q4_K / Q5_K / Q6_K 128 (qs / ql)
//   h  high bits: Q5_0 / Q5_1 the 32-bit qh word, Q5_K qh (32 bytes), Q6_K qh (64 bytes)
//   s  sub-block scales: Q4_K / Q5_K the 12 packed bytes (padded to 16), Q6_K the 16 int8 scales
//   d  the fp16 scale of every block; m the fp16 minimum (Q5_1) or dmin (Q4_K, Q5_K)
// Bytes and their meaning are unchanged, so the arithmetic on them is the reference's. One reordering: for the
// K types every group of 32 bytes indexed by an element's position j in its 32-element sub-block (Q4_K / Q5_K qs
// and qh, Q6_K ql and qh) is stored in residue order, byte j at position residue_pos(j) = 4 (j % 8) + j / 8, so
// that 32-bit word w holds elements w, w + 8, w + 16, w + 24 - the four elements that feed the reference's integer
// lane w (quant.cpp:118-144, 394-416: element e feeds lane e % 8) - and one v_dot4 gives a lane's partial sum.
// Q8_K activation quants are stored in the same order.
//
// Activations are quantized on the device into planes too: qs (int8, 32 or 256 per block), d (float: the
// block's scale, for Q8_0 / Q8_1 the fp16-rounded value widened exactly), s (float, Q8_1's fp16-rounded sum term)
// and bsums (int16 x 16 per Q8_K block).
#include <cstdint>

namespace nbh_quant {

enum Type : int { kQ4_0 = 2, kQ5_0 = 6, kQ5_1 = 7, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14 };
enum Act : int { kActQ8_0 = 0, kActQ8_1 = 1, kActQ8_K = 2 };

constexpr int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

constexpr bool is_quant(int t) {
  return t == kQ4_0 || t == kQ5_0 || t == kQ5_1 || t == kQ8_0 || t == kQ4_K || t == kQ5_K || t == kQ6_K;
}
constexpr bool is_k(int t) { return t == kQ4_K || t == kQ5_K || t == kQ6_K; }
constexpr int64_t block_elems(int t) { return is_k(t) ? 256 : 32; }
constexpr int64_t block_bytes(int t) {  // ggml block size in the file
  switch (t) {
    case kQ4_0: return 18;
    case kQ5_0: return 22;
    case kQ5_1: return 24;
    case kQ8_0: return 34;
    case kQ4_K: return 144;
    case kQ5_K: return 176;
    case kQ6_K: return 210;
    default: return 0;
  }
}
constexpr int act_of(int t) { return t == kQ5_1 ? kActQ8_1 : is_k(t) ? kActQ8_K : kActQ8_0; }

constexpr int residue_pos(int j) { return 4 * (j & 7) + (j >> 3); }

// Bytes per block in each plane (0: the plane is absent).
constexpr int64_t q_bytes(int t) { return t == kQ8_0 ? 32 : is_k(t) ? 128 : 16; }
constexpr int64_t h_bytes(int t) { return t == kQ5_0 || t == kQ5_1 ? 4 : t == kQ5_K ? 32 : t == kQ6_K ? 64 : 0; }
constexpr int64_t s_bytes(int t) { return is_k(t) ? 16 : 0; }
constexpr int64_t m_bytes(int t) { return t == kQ5_1 || t == kQ4_K || t == kQ5_K ? 2 : 0; }

// Plane offsets for `rows` rows of `nb` blocks; row r's blocks of plane p start at p_off + r * nb * p_bytes.
struct WeightLayout {
  int64_t q_off, h_off, s_off, d_off, m_off, bytes;
};
inline WeightLayout weight_layout(int t, int64_t rows, int64_t nb) {
  WeightLayout l{};
  const int64_t blocks = rows * nb;
  l.q_off = 0;
  l.h_off = align256(l.q_off + blocks * q_bytes(t));
  l.s_off = align256(l.h_off + blocks * h_bytes(t));
  l.d_off = align256(l.s_off + blocks * s_bytes(t));
  l.m_off = align256(l.d_off + blocks * 2);
  l.bytes = align256(l.m_off + blocks * m_bytes(t));
  return l;
}

// Activation planes for n rows of nb blocks of kind `act`.
struct ActLayout {
  int64_t qs_off, d_off, s_off, bsums_off, bytes;
};
inline ActLayout act_layout(int act, int64_t n, int64_t nb) {
  ActLayout l{};
  const int64_t blocks = n * nb, per = act == kActQ8_K ? 256 : 32;
  l.qs_off = 0;
  l.d_off = align256(blocks * per);
  l.s_off = align256(l.d_off + blocks * 4);
  l.bsums_off = align256(l.s_off + (act == kActQ8_1 ? blocks * 4 : 0));
  l.bytes = align256(l.bsums_off + (act == kActQ8_K ? blocks * 32 : 0));
  return l;
}

}  // namespace nbh_quant
