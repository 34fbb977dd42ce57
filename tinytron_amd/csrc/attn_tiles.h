// Tile-level building blocks shared by the decode and prefill attention
// kernels (gfx950): 16-byte K/V fragment loads through raw buffer resources
// (rows past a length read nothing), V staged straight into LDS, the QK^T /
// online-softmax step and the PV step on v_mfma_f32_16x16x32_{bf16,fp8}
// (bf16 V read back transposed from LDS with ds_read_b64_tr_b16, fp8 V
// transposed across lanes by an exact 0/1 selection MFMA), and paged block
// addressing. Everything is in an unnamed namespace: each kernel file
// gets its own copy.
#pragma once

#include "tt_internal.h"
#include "tt_numerics.h"
#include "wave_reduce.h"

namespace tt {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr float kNegInf = -__builtin_huge_valf();

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] in [15:14]).
constexpr int vmcnt_only(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }
constexpr int kLgkmcntZero = 15 | (7 << 4) | (0 << 8) | (3 << 14);

__device__ __forceinline__ int64_t uniform64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_fp8(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(__builtin_bit_cast(long, a), __builtin_bit_cast(long, b), c, 0,
                                                    0, 0);
}

// 8 e4m3fn codes -> 8 bf16 (exact).
__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(u32x2 v) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.x, 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.x, 1.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.y, 1.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.y, 1.0f, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

constexpr int kBufferFlags = 0x00020000;  // gfx9 raw buffer: dword data format, no swizzle

// Every lane loads 16 bytes per load: lane (m + 16g) reads row (token) m of a
// 16-token block at byte offset 16g + 64u, u < D*E/64. For bf16 a 16-byte
// fragment is one 32-wide k step of a 16x16x32 MFMA (d = 32u + 8g + i); for
// fp8 it is two k steps (hh = 0, 1: d = 64u + 16g + 8hh + i). The query
// operand is loaded in the same d order, so Q.K^T is unchanged.
template <bool kFP8>
struct KVTraits;

template <>
struct KVTraits<false> {
  static constexpr int kElemBytes = 2;
  static constexpr int kStepsPerFrag = 1;
  static __device__ __forceinline__ bf16x8 step(u32x4 f, int) { return __builtin_bit_cast(bf16x8, f); }
  // d of k-slot (g, i) of k step s
  static __device__ __forceinline__ int q_offset(int s, int g) { return 32 * s + 8 * g; }
};

template <>
struct KVTraits<true> {
  static constexpr int kElemBytes = 1;
  static constexpr int kStepsPerFrag = 2;
  static __device__ __forceinline__ bf16x8 step(u32x4 f, int hh) {
    return hh == 0 ? fp8x8_to_bf16x8(u32x2{f[0], f[1]}) : fp8x8_to_bf16x8(u32x2{f[2], f[3]});
  }
  static __device__ __forceinline__ int q_offset(int s, int g) { return 64 * (s >> 1) + 16 * g + 8 * (s & 1); }
};

// Row length of the cache (its head_dim) for a kernel built on D-wide tiles:
// D itself, or (kPad) the runtime head_dim a.head_dim < D (a multiple of 16
// bytes: of 8 bf16 or 16 fp8 values). Padded kernels read each cached row with
// the D-wide tile's 16-byte fragments, so a fragment that starts past the
// row's end holds the first values of the next cached token of the same 16-token
// block (the same sequence and KV head), or zero fill past the block's valid
// rows. The query's entries past head_dim are zero, so Q K^T sums the real
// head_dim only (those neighbouring values are finite unless a token this
// query attends is itself non-finite, which makes the output NaN anyway), and
// V columns past head_dim feed only output columns that are never written.
template <int D, bool kPad>
__device__ __forceinline__ int row_len(const DecodeArgs &a) {
  if constexpr (kPad) return a.head_dim;
  return D;
}

// Scale-array index of the row at element offset elem (a multiple of the row
// length): elem / head_dim, exactly (a shift for the unpadded widths; for
// padded ones a double-precision product with 1 / head_dim, rounded: the
// error is below 2^-12 for offsets under 2^40, so the nearest integer is the
// quotient).
template <int D, bool kPad>
__device__ __forceinline__ int64_t scale_row(const DecodeArgs &a, int64_t elem) {
  if constexpr (kPad) return (int64_t)__builtin_rint((double)elem * a.inv_head_dim);
  return elem / D;
}

template <int D, bool kFP8>
struct Tile {
  static constexpr int NU = D * KVTraits<kFP8>::kElemBytes / 64;  // 16-byte fragments per lane per row
  u32x4 k[2][NU];  // K fragments of the tile's two 16-token blocks (V goes through LDS)
  f32x4 ks[2];     // fp8: K scales of this lane's 4 score rows, per 16-token block
  f32x4 vs[2];
  static constexpr int kVBytes = 2 * NU * 1024;  // per-wave LDS bytes of one tile's V
};

// Element offset of token tb (a multiple of 16) of (b, hk), d = 0; tb must
// lie in a page the sequence owns. A 16-token block never straddles a page:
// paged pools have power-of-two pages of >= 16 tokens, and the contiguous
// store is addressed linearly (its pages are dense, page stride = P * D).
__device__ __forceinline__ int64_t block_elem(const DecodeArgs &a, int b, int hk, int tb, int D) {
  if (a.page_table != nullptr) {
    int64_t phys = a.page_table[(int64_t)b * a.max_pages + (tb >> a.page_shift)];
    phys = phys < 0 ? 0 : (phys >= a.num_pages ? a.num_pages - 1 : phys);
    return phys * a.c_page + (int64_t)hk * a.c_head + (int64_t)(tb & ((1 << a.page_shift) - 1)) * D;
  }
  return (int64_t)b * a.c_seq + (int64_t)hk * a.c_head + (int64_t)tb * D;
}

// Element offset of any token t < length of (b, hk), d = 0.
__device__ __forceinline__ int64_t token_elem(const DecodeArgs &a, int b, int hk, int t, int D) {
  const int tb = t & ~15;
  return block_elem(a, b, hk, tb, D) + (int64_t)(t - tb) * D;
}

// Loads of one 16-token block whose element offset `elem` was resolved in
// the prologue. Rows past the sequence end are outside the buffer range
// (num_records) and read as zero (or, for LDS loads, leave the LDS slot as
// it was): no branch, no out-of-bounds access, and no garbage (possibly
// NaN) from unused cache slots reaches the MFMAs.
template <int D, bool kFP8, bool kPad = false>
__device__ __forceinline__ void load_k_block(const DecodeArgs &a, int64_t elem, int rows, int lane,
                                             u32x4 (&k)[Tile<D, kFP8>::NU], f32x4 &ks, f32x4 &vs) {
  constexpr int E = KVTraits<kFP8>::kElemBytes;
  constexpr int NU = Tile<D, kFP8>::NU;
  const int hd = row_len<D, kPad>(a);
  const auto rk = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char *>(static_cast<const char *>(a.k_cache)) + elem * E, (short)0, rows * hd * E, kBufferFlags);
  const int off = (lane & 15) * hd * E + 16 * (lane >> 4);
#pragma unroll
  for (int u = 0; u < NU; ++u)
    k[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off + 64 * u, 0, 0));
  if constexpr (kFP8) {
    // this lane's score rows are tokens tb + 4g + r, r = 0..3
    // the block starts a 16-row scale group (the host checks the strides), so
    // its K and V scales are 16 consecutive entries of each array
    const int64_t sidx = fp8_scale_index(scale_row<D, kPad>(a, elem));
    const auto rks = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.k_scale) + sidx, (short)0,
                                                       rows * 4, kBufferFlags);
    const auto rvs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.v_scale) + sidx, (short)0,
                                                       rows * 4, kBufferFlags);
    ks = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rks, 16 * (lane >> 4), 0, 0));
    vs = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rvs, 16 * (lane >> 4), 0, 0));
  }
}

// V rows of one 16-token block straight into this wave's LDS slots
// (buffer_load ... lds: lane i's 16 bytes land at base + 16 i, the layout a
// register load would have), so the next tile's V costs no VGPRs.
template <int D, bool kFP8, bool kPad = false>
__device__ __forceinline__ void load_v_block_lds(const DecodeArgs &a, int64_t elem, int rows, int lane, char *lds) {
  constexpr int E = KVTraits<kFP8>::kElemBytes;
  constexpr int NU = Tile<D, kFP8>::NU;
  const int hd = row_len<D, kPad>(a);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char *>(static_cast<const char *>(a.v_cache)) + elem * E, (short)0, rows * hd * E, kBufferFlags);
  // bf16 slots are swizzled for read_v's transposing reads: slot m + 16 g
  // holds token m ^ (8 (g & 1)) (chunk g), so that the two 8-column chunks
  // that one read takes from each of 8 tokens fill all 64 banks once
  const int tok = kFP8 ? (lane & 15) : ((lane & 15) ^ (8 * ((lane >> 4) & 1)));
  const int off = tok * hd * E + 16 * (lane >> 4);
#pragma unroll
  for (int u = 0; u < NU; ++u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void *)(lds + 1024 * u), 16,
                                             off + 64 * u, 0, 0, 0);
}

template <int D, bool kFP8>
struct WaveState {
  static constexpr int NDB = D / 32;
  f32x4 o[2 * NDB];  // PV accumulators, transposed: block c, lane (n + 16g) = column n, d = o_col_d(c, 4g + r)
  float m;           // running max of this lane's head (log2 units)
  float l;           // running sum (lane-partial: this lane's tokens only)
};

template <int D, bool kFP8>
__device__ __forceinline__ void qk_softmax(float scale_log2, int t0, int lim, int lane, const Tile<D, kFP8> &tile,
                                           const bf16x8 (&qf)[D / 32], WaveState<D, kFP8> &st, bf16x8 &pa_hi,
                                           bf16x8 &pa_lo) {
  using TR = KVTraits<kFP8>;
  constexpr int NDB = D / 32;
  const int g = lane >> 4;

  // S^T[token][head]: lane (n + 16g), reg r = token t0 + 16*tt + 4g + r, head n.
  f32x4 S[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    S[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NDB; ++s) {
      const int u = s / TR::kStepsPerFrag;
      S[tt] = mfma_bf16(TR::step(tile.k[tt][u], s % TR::kStepsPerFrag), qf[s], S[tt]);
    }
  }

  float s[8];
  bool valid[8];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = t0 + 16 * tt + 4 * g + r;
      float x = S[tt][r];
      if constexpr (kFP8) x *= tile.ks[tt][r];
      valid[tt * 4 + r] = tok < lim;
      s[tt * 4 + r] = tok < lim ? x * scale_log2 : kNegInf;
    }
  }
  // maxima: IEEE-754-2019 maximum (no score is NaN; masked ones are -inf), the
  // nested pairs folding into v_maximum3_f32; across the four lane groups with
  // permlane swaps (with both operands x, the two results' maximum is the
  // maximum of x[lane] and x[lane ^ 16], resp. x[lane ^ 32])
  const auto mx2 = [](float u, float v) { return __builtin_elementwise_maximum(u, v); };
  float mx = mx2(mx2(mx2(mx2(s[0], s[1]), s[2]), mx2(mx2(s[3], s[4]), s[5])), mx2(s[6], s[7]));
  const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
  mx = mx2(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
  const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
  mx = mx2(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
  const float m_new = mx2(st.m, mx);  // finite: every column has key t0 = 0 valid from its first tile on
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
  float p[8];
  float psum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    p[i] = __builtin_amdgcn_exp2f(s[i] - m_new);
    psum += p[i];
  }
  st.l = st.l * alpha + psum;
  st.m = m_new;
  if constexpr (kFP8) {
    // fold the per-token V scale into P; masked tokens stay exactly 0 (select,
    // not multiply, in case a scale slot past the end holds a non-finite value)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = valid[r] ? p[r] * tile.vs[0][r] : 0.f;
      p[4 + r] = valid[4 + r] ? p[4 + r] * tile.vs[1][r] : 0.f;
    }
  }

  // O is held transposed (see pv_tile): every value of a lane is in the
  // lane's own column, rescaled by its own alpha.
#pragma unroll
  for (int c = 0; c < 2 * NDB; ++c) st.o[c] *= alpha;

  // P as the A operand: row = head (lane % 16), k slots = this lane's 8 tokens.
  // P = P_hi + P_lo with both halves bf16 (P_lo = P - P_hi is exact in fp32),
  // so the PV product keeps ~16 mantissa bits of P instead of bf16's 8; the
  // second MFMA per block is free in this memory-bound loop.
  const f32x8 pv = {p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]};
  pa_hi = __builtin_convertvector(pv, bf16x8);
  const f32x8 p_rem = pv - __builtin_convertvector(pa_hi, f32x8);
  pa_lo = __builtin_convertvector(p_rem, bf16x8);
}


// A tile's V for the PV product, read from its LDS slot (the two 16-token
// blocks' fragments at slot + (tt * NU + u) * 1024 + lane * 16, as
// load_v_block_lds lays them out). fp8 keeps the raw fragments, transposed on
// the matrix cores inside pv_tile. bf16 reads each 16-column block already
// transposed with ds_read_b64_tr_b16: in every group of 16 lanes, lane i
// receives element i % 4 of the 8-byte rows that lanes 4j + i / 4 address,
// j = 0..3, as its elements j (lane layout measured on gfx950). Lane s =
// 4j + q of group g addresses token 4g + j, columns 16c + 4q .. + 3, so lane
// (n + 16g) gets V[16h + 4g + j][16c + n] for j < 4 -- h = 0 its elements
// 0-3, h = 1 its elements 4-7 -- the PV MFMA's B operand in the token order
// of the P operand (the same values the selection MFMA produced, with no
// MFMA and no conversion).
template <int D, bool kFP8>
struct VRegs;
template <int D>
struct VRegs<D, true> {
  u32x4 vt[2][Tile<D, true>::NU];
};
template <int D>
struct VRegs<D, false> {
  bf16x8 vb[D / 16];
};

template <int D, bool kFP8>
__device__ __forceinline__ void read_v(const char *vlds, int lane, VRegs<D, kFP8> &v) {
  constexpr int NU = Tile<D, kFP8>::NU;
  if constexpr (kFP8) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int u = 0; u < NU; ++u) v.vt[tt][u] = *reinterpret_cast<const u32x4 *>(vlds + (tt * NU + u) * 1024 + lane * 16);
  } else {
    typedef __bf16 bf16x4v __attribute__((ext_vector_type(4)));
    const int row = 4 * (lane >> 4) + ((lane >> 2) & 3);  // token 4g + j of each 16-token block
    const int q = lane & 3;                                  // columns 4q .. 4q + 3 of the 16-column block
    const int slot = row ^ (8 * (q >> 1));                   // the swizzled slot of load_v_block_lds
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      bf16x4v part[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int byte = (h * NU + (c >> 1)) * 1024 + (slot + 16 * (2 * (c & 1) + (q >> 1))) * 16 + 8 * (q & 1);
        part[h] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (__attribute__((address_space(3))) bf16x4v *)(vlds + byte));
      }
      v.vb[c] = bf16x8{part[0][0], part[0][1], part[0][2], part[0][3], part[1][0], part[1][1], part[1][2], part[1][3]};
    }
  }
}

// V^T of block c (16 output columns o_col_d(c, n)): lane (n + 16g) holds
// V[token t0 + 4g + r][col] (elements r < 4) and V[t0 + 16 + 4g + r][col]
// (elements 4 + r), as bf16.
template <int D, bool kFP8>
__device__ __forceinline__ bf16x8 v_block(const VRegs<D, kFP8> &v, int c, const u32x2 (&ident8)[2]) {
  if constexpr (kFP8) {
    // block c = 4u + 2hh + hi (column order in o_col_d): the fp8 fragments
    // transposed by an exact 0/1 selection MFMA
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const int hi = c & 1, u = c >> 2, hh = (c >> 1) & 1;
    const u32x2 v0 = hh ? u32x2{v.vt[0][u][2], v.vt[0][u][3]} : u32x2{v.vt[0][u][0], v.vt[0][u][1]};
    const u32x2 v1 = hh ? u32x2{v.vt[1][u][2], v.vt[1][u][3]} : u32x2{v.vt[1][u][0], v.vt[1][u][1]};
    const f32x4 t0v = mfma_fp8(v0, ident8[hi], zero);
    const f32x4 t1v = mfma_fp8(v1, ident8[hi], zero);
    const f32x8 vv = {t0v[0], t0v[1], t0v[2], t0v[3], t1v[0], t1v[1], t1v[2], t1v[3]};
    return __builtin_convertvector(vv, bf16x8);
  } else {
    return v.vb[c];
  }
}

// PV of one tile, accumulated transposed: O^T = V^T P^T, the V block as the
// A operand and P_hi / P_lo as B (the registers P V would use, operands
// swapped). Lane (n + 16g) holds O^T[d][column n] for d = o_col_d(c, 4g + r),
// r = 0..3: a lane's values all belong to its own column (no cross-lane
// rescale), four consecutive head_dim entries per block.
template <int D, bool kFP8>
__device__ __forceinline__ void pv_tile(const VRegs<D, kFP8> &v, const u32x2 (&ident8)[2], bf16x8 pa_hi,
                                        bf16x8 pa_lo, WaveState<D, kFP8> &st) {
  constexpr int NDB = D / 32;
#pragma unroll
  for (int c = 0; c < 2 * NDB; ++c) {
    const bf16x8 vb = v_block<D, kFP8>(v, c, ident8);
    st.o[c] = mfma_bf16(vb, pa_hi, st.o[c]);
    st.o[c] = mfma_bf16(vb, pa_lo, st.o[c]);
  }
}

// head_dim index of output column n of PV block c (see pv_tile).
template <bool kFP8>
__device__ __forceinline__ int o_col_d(int c, int n) {
  if constexpr (kFP8) {
    const int u = c >> 2, hh = (c >> 1) & 1, hi = c & 1;
    return 64 * u + 16 * (2 * hi + (n >> 3)) + 8 * hh + (n & 7);
  } else {
    return 16 * c + n;
  }
}

// Selection matrices for the V transpose: B[k][n] = 1 iff k == n (+16 for
// the upper half), expressed in the (lane group, slot) coordinates in which
// the A operand was loaded, so the result does not depend on how the
// hardware orders the K index inside a lane.
__device__ __forceinline__ void make_identity(int lane, bf16x8 (&ident16)[2], u32x2 (&ident8)[2]) {
  const int n = lane & 15;
  const int g = lane >> 4;
  uint32_t w8[2][2] = {{0u, 0u}, {0u, 0u}};
  uint32_t w16[2][4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (8 * g + i == n) {
      w8[0][i >> 2] |= 0x38u << (8 * (i & 3));        // e4m3fn 1.0
      w16[0][i >> 1] |= 0x3f80u << (16 * (i & 1));    // bf16 1.0
    }
    if (8 * g + i == n + 16) {
      w8[1][i >> 2] |= 0x38u << (8 * (i & 3));
      w16[1][i >> 1] |= 0x3f80u << (16 * (i & 1));
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    ident8[h] = u32x2{w8[h][0], w8[h][1]};
    ident16[h] = __builtin_bit_cast(bf16x8, u32x4{w16[h][0], w16[h][1], w16[h][2], w16[h][3]});
  }
}

constexpr int kChunkTiles = 16;  // tiles per page-table fetch and software-pipelined run (<= 64 pages of 16 tokens)

// Element offset and valid rows of 16-token block `blk` of (b, hk). Paged:
// `entry` holds, one per lane, the page-table entries of pages pbase.. (the
// block's page index relative to pbase is < 64 for every block of the chunk).
template <int D, bool kPad = false>
__device__ __forceinline__ void stream_block_addr(const DecodeArgs &a, int b, int hk, int L, int entry, int pbase,
                                                  int blk, int64_t &elem, int &rows) {
  const int hd = row_len<D, kPad>(a);
  const int tb = 16 * blk;
  const int tc = min(tb, (L - 1) & ~15);  // blocks past the end keep an in-sequence address and zero rows
  rows = __builtin_amdgcn_readfirstlane(min(max(L - tb, 0), 16));
  int64_t e;
  if (a.page_table != nullptr) {
    int64_t phys = __builtin_amdgcn_readlane(entry, (tc >> a.page_shift) - pbase);
    phys = phys < 0 ? 0 : (phys >= a.num_pages ? a.num_pages - 1 : phys);
    e = phys * a.c_page + (int64_t)hk * a.c_head + (int64_t)(tc & ((1 << a.page_shift) - 1)) * hd;
  } else {
    e = (int64_t)b * a.c_seq + (int64_t)hk * a.c_head + (int64_t)tc * hd;
  }
  elem = uniform64(e);
}


}  // namespace
}  // namespace tt
