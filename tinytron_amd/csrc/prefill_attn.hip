// Prefill GQA attention for gfx950: T new tokens per sequence attend causally
// to their sequence's cached keys (the prompt chunk's own K/V already
// appended by rope_append), over the reference's contiguous store or the
// paged pool, bf16 or fp8-e4m3 cache.
//
// Replaces the prefill branch of the reference's attention (attn.py:321-341:
// append, get_kv, then SDPA with is_causal=True at past_len 0 or the mask
// key_pos <= past_len + query_pos otherwise) for a ragged batch.
//
// One wave per (sequence b, KV head hk, NB consecutive blocks of qt = 16 / G
// query tokens): the 16 columns of a block's MFMA B operand are the (token,
// head) pairs n = tq * G + head, so each streamed K/V tile serves G heads x
// NB * qt tokens (the tile's K fragments and its transposed V are reused by
// all NB blocks). The key loop is the decode kernel's tile pipeline (K
// fragments in registers, V through LDS, QK^T and PV on the matrix cores,
// online softmax per column); column n masks the keys after its own position
// (position 0 is valid for every column, so no row is ever empty).
//
// Workgroups are laid out so that all query blocks of one (sequence, KV
// head) go to the same XCD (workgroup i runs on XCD i mod 8): the pair's
// K/V, re-read by each of its blocks, stays in that XCD's L2.
#include <algorithm>

#include "attn_tiles.h"
#include "tt_internal.h"
#include "tt_numerics.h"

namespace tt {
namespace {

constexpr int kXcds = 8;
// Tiles per page-table fetch and pipelined run: 8 here (16 measured 25 %
// slower: NB column blocks per wave already make the unrolled body long).
constexpr int kPrefillChunkTiles = 8;

// QK^T and the online-softmax step of one 32-token tile for one column block
// (16 (token, head) columns). Unlike the decode step this loop is bound by
// VALU issue, so: bf16 scores become y = s * scale - m in one FMA; the causal
// mask runs only on `edge` tiles (those reaching past the smallest limit of
// the wave's columns: every other tile is whole for every column); the
// maximum is the IEEE-754-2019 one (v_maximum3_f32, which needs no NaN
// quieting of its inputs; no score is NaN). P enters PV as P_hi + P_lo
// (two bf16 operands, ~16 mantissa bits: a single bf16 P misses the 2e-3
// absolute bound on short, cancelling rows). The running max is lazy: a
// column's reference max st.m moves only when the tile's max exceeds it by
// more than kLazyMax (log2 units), so P <= 2^kLazyMax (fp32 O and l and the
// bf16 P halves have the range) and most tiles need no rescale at all.
// Returns whether any column of the wave moved its max; then the caller
// rescales O by `alpha` (this column's exp2(m_old - m_new), 1 for columns
// that kept theirs, 0 on the first tile, whose key 0 is valid for every
// column).
constexpr float kLazyMax = 8.0f;
template <int D, bool kFP8>
__device__ __forceinline__ bool qk_softmax_pf(float scale_log2, const f32x4 (&kc)[2], bool edge, int t0, int lim,
                                              int lane, const Tile<D, kFP8> &tile, const bf16x8 (&qf)[D / 32],
                                              WaveState<D, kFP8> &st, float &alpha, bf16x8 &pa_hi, bf16x8 &pa_lo) {
  using TR = KVTraits<kFP8>;
  constexpr int NDB = D / 32;
  const int g = lane >> 4;
  // S^T[token][column]: lane (n + 16g), reg r = token t0 + 16*tt + 4g + r, column n.
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
  // x: raw scores (bf16) or scores in log2 units (fp8: K scale x softmax scale)
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = kFP8 ? S[i >> 2][i & 3] * kc[i >> 2][i & 3] : S[i >> 2][i & 3];
  if (edge) {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = t0 + 16 * (i >> 2) + 4 * g + (i & 3) < lim ? x[i] : kNegInf;
  }
  const auto mx2 = [](float u, float v) { return __builtin_elementwise_maximum(u, v); };
  // nested pairs fold into three-input v_maximum3_f32 (four instructions for eight values)
  float mx = mx2(mx2(mx2(mx2(x[0], x[1]), x[2]), mx2(mx2(x[3], x[4]), x[5])), mx2(x[6], x[7]));
  // The reference max moves only past the slack (always on the first tile:
  // st.m = -inf). A column moves iff one of its four lanes' own maxima is past
  // it (scaling by scale > 0 and rounding keep the order, -inf stays -inf), so
  // the maxima across the lane groups need only be formed when some column
  // moves (same results).
  const bool lane_past = (kFP8 ? mx : mx * scale_log2) > st.m + kLazyMax;
  const bool rescale = __builtin_amdgcn_ballot_w64(lane_past) != 0;  // wave-uniform
  alpha = 1.0f;
  float m_new = st.m;
  if (rescale) {  // across the four lane groups (lanes n, n+16, n+32, n+48 hold column n)
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = mx2(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = mx2(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
    if constexpr (!kFP8) mx *= scale_log2;
    m_new = mx > st.m + kLazyMax ? mx : st.m;
    alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.m = m_new;
  }
  float p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    p[i] = __builtin_amdgcn_exp2f(kFP8 ? x[i] - m_new : __builtin_fmaf(x[i], scale_log2, -m_new));
  if constexpr (kFP8) {  // bf16: the column sums come from the matrix cores (see pv_block)
    const float psum = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    st.l = rescale ? __builtin_fmaf(st.l, alpha, psum) : st.l + psum;
  }
  if constexpr (kFP8) {
    // fold the per-token V scale into P; on edge tiles masked tokens stay
    // exactly 0 (select: a scale slot past the end may hold anything)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float pv = p[i] * tile.vs[i >> 2][i & 3];
      p[i] = edge ? (p[i] == 0.f ? 0.f : pv) : pv;
    }
  }
  const f32x8 pv = {p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]};
  pa_hi = __builtin_convertvector(pv, bf16x8);
  // P_hi back in fp32 straight from the packed halves (element 2i is the low half of word i)
  const u32x4 hw = __builtin_bit_cast(u32x4, pa_hi);
  f32x8 hf;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hf[2 * i] = __uint_as_float(hw[i] << 16);
    hf[2 * i + 1] = __uint_as_float(hw[i] & 0xffff0000u);
  }
  pa_lo = __builtin_convertvector(pv - hf, bf16x8);  // P - P_hi exact in fp32
  return rescale;
}

// PV of one tile for one column block, accumulated transposed: Oᵀ = Vᵀ Pᵀ,
// with the V block as the A operand and P_hi + P_lo as B (the same
// registers as in P V: lane (n + 16g) holds V[tokens of group g][d n] and
// P[column n][tokens of group g]). Lane (n + 16g) then holds Oᵀ[d][column n]
// for d = o_col_d(c, 4g + r): every O value of a lane belongs to its own
// column, so the rescale by alpha needs no cross-lane traffic, and each
// block's four values are consecutive head_dim entries. bf16 caches also
// accumulate the softmax denominators here: an all-ones A block gives every
// column's sum of P_hi + P_lo in each of its lanes (two MFMAs instead of
// eight VALU adds per block and tile, in a loop bound by VALU issue; fp8 P
// carries the V scales, so fp8 sums on the VALU). `vb` are the tile's V
// blocks (v_block), converted once for all column blocks.
template <int D, bool kFP8>
__device__ __forceinline__ void pv_block(const bf16x8 (&vb)[D / 16], bf16x8 pa_hi, bf16x8 pa_lo,
                                         WaveState<D, kFP8> &st, f32x4 &lsum) {
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    st.o[c] = mfma_bf16(vb[c], pa_hi, st.o[c]);
    st.o[c] = mfma_bf16(vb[c], pa_lo, st.o[c]);
  }
  if constexpr (!kFP8) {
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
    lsum = mfma_bf16(ones, pa_hi, lsum);
    lsum = mfma_bf16(ones, pa_lo, lsum);
  }
}

// Column blocks per wave and workgroups per CU. bf16 at head_dim 128 runs
// 4 blocks at one workgroup per CU (up to 512 registers a wave): the K
// fragments and transposed V of a tile then feed twice the MFMA work per
// byte read, which pays more than the second workgroup's latency hiding.
// fp8 keeps 2 blocks at two workgroups per CU at 128: its dequantisation is
// VALU work that needs the second workgroup to hide.
template <int D, bool kFP8>
constexpr int prefill_blocks() {
  return D <= 64 ? 4 : (kFP8 ? 2 : 4);
}

template <int D, bool kFP8>
constexpr int prefill_wgs_per_cu() {
  return (D == 128 && !kFP8) ? 1 : 2;
}

template <int D, bool kFP8, int NB, bool kPad>
__global__ __launch_bounds__(256, (prefill_wgs_per_cu<D, kFP8>())) void prefill_attn_kernel(PrefillArgs a) {
  using TR = KVTraits<kFP8>;
  const int hd = row_len<D, kPad>(a);
  constexpr int NDB = D / 32;
  constexpr int NU = Tile<D, kFP8>::NU;
  constexpr int kKLoads = 2 * NU + (kFP8 ? 4 : 0);
  constexpr int kVAll = kWavesPerBlock * Tile<D, kFP8>::kVBytes;
  extern __shared__ char smem_v[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int i = threadIdx.x; i < kVAll / 16; i += 64 * kWavesPerBlock)  // the block size (not a dispatch load)
    reinterpret_cast<u32x4 *>(smem_v)[i] = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();

  // workgroup -> (XCD, slot on that XCD) -> (pair, its k-th workgroup); the
  // longest (last) query blocks of a pair go first. a.nq counts groups of NB
  // blocks here.
  const int xcd = blockIdx.x % kXcds;
  const int slot = blockIdx.x / kXcds;
  const int pair = (slot / a.wg_per_pair) * kXcds + xcd;
  if (pair >= a.batch * a.hkv) return;
  const int qgrp = a.nq - 1 - ((slot % a.wg_per_pair) * kWavesPerBlock + wave);
  if (qgrp < 0) return;
  const int b = pair / a.hkv;
  const int hk = pair - b * a.hkv;
  const int nb = a.new_lens != nullptr ? min(max(a.new_lens[b], 0), a.num_new) : a.num_new;
  const int t_first = qgrp * a.qt * NB;
  if (t_first >= nb) return;
  const int pos0 = a.positions[b];
  const int t_end = min(t_first + a.qt * NB, nb);
  // keys the group needs: 0 .. pos0 + t_end - 1, never past the host's bound (the page table's reach)
  const int L = __builtin_amdgcn_readfirstlane(min(pos0 + t_end, a.max_len));
  if (pos0 < 0 || L <= 0) return;
  // smallest key limit of the wave's valid columns (its first token's): tiles
  // below it are whole for every column and skip the mask
  const int lim_min = __builtin_amdgcn_readfirstlane(min(pos0 + t_first + 1, L));

  const int G = a.group;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int tq = n / G;
  const int head = n - tq * G;
  int lim[NB];
  bf16x8 qf[NB][NDB];
  const uint16_t *q = static_cast<const uint16_t *>(a.q);
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int tb = t_first + j * a.qt;
    const bool col_valid = tq < a.qt && tb + tq < t_end;
    lim[j] = col_valid ? min(pos0 + tb + tq + 1, L) : 1;  // keys this column may see
    const int64_t qrow = (int64_t)b * a.q_sb + (int64_t)(hk * G + head) * a.q_sh + (int64_t)(tb + tq) * a.q_st;
#pragma unroll
    for (int s = 0; s < NDB; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (col_valid && (!kPad || TR::q_offset(s, g) < hd)) v = *reinterpret_cast<const u32x4 *>(q + qrow + TR::q_offset(s, g));
      qf[j][s] = __builtin_bit_cast(bf16x8, v);
    }
  }
  bf16x8 ident16[2];
  u32x2 ident8[2];
  make_identity(lane, ident16, ident8);
  WaveState<D, kFP8> st[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
#pragma unroll
    for (int c = 0; c < 2 * NDB; ++c) st[j].o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    st[j].m = kNegInf;
    st[j].l = 0.f;
  }
  f32x4 lsum[NB];  // bf16: every element holds the lane's column sum of P (rescaled with O)
#pragma unroll
  for (int j = 0; j < NB; ++j) lsum[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  char *vlds = smem_v + wave * Tile<D, kFP8>::kVBytes;
  const int ntiles = (L + kTileTokens - 1) / kTileTokens;
  // Same chunked pipeline as the decode kernel (K(k+1) | QK, softmax |
  // wait V(k), read V(k) | V(k+1) | PV), with explicit vmcnt counts.
  for (int c0 = 0; c0 < ntiles; c0 += kPrefillChunkTiles) {
    const int c1 = min(ntiles, c0 + kPrefillChunkTiles);
    int entry = 0, pbase = 0;
    if (a.page_table != nullptr) {
      pbase = (kTileTokens * c0) >> a.page_shift;
      const int last = (L - 1) >> a.page_shift;
      entry = a.page_table[(int64_t)b * a.max_pages + min(pbase + lane, last)];
    }
    Tile<D, kFP8> buf[2];
    int64_t e0, e1;
    int r0, r1;
    stream_block_addr<D, kPad>(a, b, hk, L, entry, pbase, 2 * c0, e0, r0);
    stream_block_addr<D, kPad>(a, b, hk, L, entry, pbase, 2 * c0 + 1, e1, r1);
    load_k_block<D, kFP8, kPad>(a, e0, r0, lane, buf[0].k[0], buf[0].ks[0], buf[0].vs[0]);
    load_k_block<D, kFP8, kPad>(a, e1, r1, lane, buf[0].k[1], buf[0].ks[1], buf[0].vs[1]);
    __builtin_amdgcn_sched_barrier(0);
    load_v_block_lds<D, kFP8, kPad>(a, e0, r0, lane, vlds);
    load_v_block_lds<D, kFP8, kPad>(a, e1, r1, lane, vlds + NU * 1024);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < kPrefillChunkTiles; ++k) {
      const int it = c0 + k;
      if (it >= c1) break;  // uniform
      if (k + 1 < kPrefillChunkTiles) {
        stream_block_addr<D, kPad>(a, b, hk, L, entry, pbase, 2 * it + 2, e0, r0);
        stream_block_addr<D, kPad>(a, b, hk, L, entry, pbase, 2 * it + 3, e1, r1);
        Tile<D, kFP8> &nx = buf[(k + 1) & 1];
        load_k_block<D, kFP8, kPad>(a, e0, r0, lane, nx.k[0], nx.ks[0], nx.vs[0]);
        load_k_block<D, kFP8, kPad>(a, e1, r1, lane, nx.k[1], nx.ks[1], nx.vs[1]);
      }
      __builtin_amdgcn_sched_barrier(0);
      const int t0 = kTileTokens * it;
      const bool edge = t0 + kTileTokens > lim_min;  // uniform
      f32x4 kc[2] = {};
      if constexpr (kFP8) {
        kc[0] = buf[k & 1].ks[0] * a.scale_log2;
        kc[1] = buf[k & 1].ks[1] * a.scale_log2;
      }
      // Every column block's QKᵀ and softmax go before the wait for V(k) (time
      // for its DMA to land; moving some blocks after it, to overlap their
      // softmax with other blocks' PV, measured no faster with a bf16 cache and
      // far slower with fp8 at head_dim 128). After the V read, each block's
      // rescale and PV follow with no scheduling barrier between blocks.
      bf16x8 pa_hi[NB], pa_lo[NB];
      float alpha[NB];
      bool rescale[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j)
        rescale[j] = qk_softmax_pf<D, kFP8>(a.scale_log2, kc, edge, t0, lim[j], lane, buf[k & 1], qf[j], st[j],
                                            alpha[j], pa_hi[j], pa_lo[j]);
      __builtin_amdgcn_sched_barrier(0);
      if (k + 1 < kPrefillChunkTiles)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(kKLoads));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
      VRegs<D, kFP8> vr;
      read_v<D, kFP8>(vlds, lane, vr);
      __builtin_amdgcn_s_waitcnt(kLgkmcntZero);
      __builtin_amdgcn_sched_barrier(0);
      if (k + 1 < kPrefillChunkTiles && it + 1 < c1) {
        load_v_block_lds<D, kFP8, kPad>(a, e0, r0, lane, vlds);
        load_v_block_lds<D, kFP8, kPad>(a, e1, r1, lane, vlds + NU * 1024);
      }
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 vb[D / 16];
#pragma unroll
      for (int c = 0; c < D / 16; ++c) vb[c] = v_block<D, kFP8>(vr, c, ident8);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        // every Oᵀ value of a lane is in the lane's own column: its own alpha
        if (rescale[j]) {  // uniform
#pragma unroll
          for (int c = 0; c < 2 * NDB; ++c) st[j].o[c] *= alpha[j];
          if constexpr (!kFP8) lsum[j] *= alpha[j];
        }
        pv_block<D, kFP8>(vb, pa_hi[j], pa_lo[j], st[j], lsum[j]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
  }

  // normalise and write: lane (n + 16g) holds column n's head_dim entries
  // o_col_d(c, 4g) .. + 3 of every block c
  uint16_t *out = static_cast<uint16_t *>(a.out);
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int tb = t_first + j * a.qt;
    float l = lsum[j][0];
    if constexpr (kFP8) {
      l = st[j].l;
      l += __shfl_xor(l, 16, 64);
      l += __shfl_xor(l, 32, 64);
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    if (tq < a.qt && tb + tq < t_end) {
      const int64_t orow = (int64_t)b * a.o_sb + (int64_t)(tb + tq) * a.o_st + (int64_t)(hk * G + head) * a.o_sh;
#pragma unroll
      for (int c = 0; c < 2 * NDB; ++c) {
        const int d0 = o_col_d<kFP8>(c, 4 * g);
        if (kPad && d0 >= hd) continue;  // columns past head_dim (hd is a multiple of 8)
        const uint2 w = make_uint2(pack_bf16x2(st[j].o[c][0] * inv, st[j].o[c][1] * inv),
                                   pack_bf16x2(st[j].o[c][2] * inv, st[j].o[c][3] * inv));
        if (a.vec_out) {
          *reinterpret_cast<uint2 *>(out + orow + d0) = w;
        } else {
          out[orow + d0] = (uint16_t)w.x;
          out[orow + d0 + 1] = (uint16_t)(w.x >> 16);
          out[orow + d0 + 2] = (uint16_t)w.y;
          out[orow + d0 + 3] = (uint16_t)(w.y >> 16);
        }
      }
    }
  }
}

template <int D, bool kFP8, bool kPad>
hipError_t launch_d(const PrefillArgs &a0, hipStream_t stream) {
  constexpr int NB = prefill_blocks<D, kFP8>();
  PrefillArgs a = a0;
  a.nq = (a0.nq + NB - 1) / NB;  // groups of NB query blocks
  a.wg_per_pair = (a.nq + kWavesPerBlock - 1) / kWavesPerBlock;
  const int64_t pairs = (int64_t)a.batch * a.hkv;
  const int64_t slots = (pairs + kXcds - 1) / kXcds * a.wg_per_pair;
  const int64_t grid = slots * kXcds;
  const size_t lds = (size_t)kWavesPerBlock * Tile<D, kFP8>::kVBytes;
  hipLaunchKernelGGL((prefill_attn_kernel<D, kFP8, NB, kPad>), dim3((unsigned)grid), dim3(64 * kWavesPerBlock), lds,
                     stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_attn(const PrefillArgs &a, CacheKind kind, int head_dim, hipStream_t stream) {
  const int D = tile_head_dim(head_dim, kind);
  const bool pad = D != head_dim;
  if (kind == CacheKind::kFP8) {
    if (D == 64) return pad ? launch_d<64, true, true>(a, stream) : launch_d<64, true, false>(a, stream);
    if (D == 128) return pad ? launch_d<128, true, true>(a, stream) : launch_d<128, true, false>(a, stream);
    return hipErrorInvalidValue;
  }
  if (D == 32) return pad ? launch_d<32, false, true>(a, stream) : launch_d<32, false, false>(a, stream);
  if (D == 64) return pad ? launch_d<64, false, true>(a, stream) : launch_d<64, false, false>(a, stream);
  if (D == 128) return pad ? launch_d<128, false, true>(a, stream) : launch_d<128, false, false>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace tt
