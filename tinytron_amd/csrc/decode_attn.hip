// GQA split-K decode attention for gfx950 (CDNA4).
//
// Computes, for one new token per sequence, what the reference computes with
// repeat_interleave + F.scaled_dot_product_attention over the cached keys
// (attn.py:66-83, 420-423): out[b, h] = softmax(q[b,h] . K_b^T * scale) V_b
// with K/V read from KV head h / G (G = H_q / H_kv).
//
// Work decomposition
//   grid = (H_kv, splits, B); one workgroup = 4 waves = one (b, kv head,
//   split) of `split_tokens` tokens; each wave streams a quarter of the split
//   in 32-token tiles and keeps an online-softmax state for the G query heads
//   of the group, so every K/V byte is read from HBM once for all G heads.
//   The 4 wave states merge in LDS into one partial per split; a second
//   kernel merges the splits of a (b, q head).
//
// Per 32-token tile, on the matrix cores (v_mfma_f32_16x16x32_bf16):
//   QK^T: A = 16 K rows (16-byte loads, one token per lane%16), B = q^T with
//         the group's heads as columns -> S^T[token][head].
//   V^T : the PV product contracts over tokens, but a 16-byte load gives a
//         lane 8 head_dim values of one token. bf16 V goes into LDS by DMA
//         (buffer_load ... lds) and comes back transposed with
//         ds_read_b64_tr_b16; fp8 V is transposed on the fp8 MFMA by a 0/1
//         selection matrix (exact: one nonzero product per output).
//   PV  : accumulated transposed, O^T = V^T P^T (A = the V^T block, B = P as a
//         bf16 hi + lo pair), so every O value a lane holds belongs to its own
//         head and the online-softmax rescale needs no cross-lane traffic.
// The token order inside a tile is the one the MFMA output layout produces,
// used consistently for S, P and V^T; the only cross-lane steps are the head
// max across the four lane groups (permlane swaps) and the final sums.
//
// fp8-e4m3fn caches: K codes become bf16 with v_cvt_scalef32_pk_bf16_fp8
// (exact: every e4m3 value is a bf16 value), the per-token K scale multiplies
// the score, the V transpose runs on the fp8 MFMA with an fp8 identity
// (exact), and the per-token V scale multiplies P before its bf16 rounding.
//
// Tokens past a sequence's length are never loaded (predicated loads, zero
// fill) and their scores are set to -inf, so garbage or NaN in unused cache
// slots cannot reach the output.
#include <algorithm>

#include "attn_tiles.h"
#include "rope_math.h"
#include "tt_internal.h"
#include "tt_numerics.h"

namespace tt {
namespace {
// Threads of every 4-wave kernel here (all but the paired one). Loops stride
// by this constant rather than blockDim.x: that is a global load from the
// dispatch's arguments (~1 us at kernel start, ahead of the first loop).
constexpr int kBlockThreads = 64 * kWavesPerBlock;

// floats of the LDS merge area: [4][G][D] outputs, [4][16] maxima, [4][16] sums
__host__ __device__ constexpr int merge_floats(int G, int D) { return kWavesPerBlock * G * D + 2 * kWavesPerBlock * 16; }

// One split of one (sequence, KV head): the 4 waves of the workgroup each
// stream kTiles 32-token tiles, merge their states in LDS and write one
// partial (unnormalised output, max, sum) to the workspace.
template <int D, bool kFP8, int kTiles, bool kPad>
__device__ __forceinline__ void split_item(const DecodeArgs &a, int b, int hk, int split, int L, int lane, int wave,
                                           char *smem_v, float *smem) {
  using TR = KVTraits<kFP8>;
  constexpr int NDB = D / 32;
  const int hd = row_len<D, kPad>(a);
  constexpr int kWaveTokens = kTiles * kTileTokens;
  constexpr int kBlocks = 2 * kTiles;  // 16-token blocks per wave
  const int G = a.group;
  const int s_begin = split * (kWavesPerBlock * kWaveTokens);
  const int w_begin = s_begin + wave * kWaveTokens;
  const int n = lane & 15;
  const int g = lane >> 4;

  // Resolve every block's address up front (page-table reads are scalar and
  // independent), so the streaming loop below has no dependent loads.
  // Blocks past the end keep a valid in-sequence token for the lookup and
  // zero rows.
  int64_t belem[kBlocks];
  int brows[kBlocks];
  if (a.page_table != nullptr) {
    // one load for the whole wave: lane i fetches the entry of the wave's
    // i-th page (clamped to the sequence's last page), then each block reads
    // its entry with v_readlane into scalar registers.
    const int j_first = min(w_begin, L - 1) >> a.page_shift;
    const int j_last = (L - 1) >> a.page_shift;
    const int pmask = (1 << a.page_shift) - 1;
    int entry = 0;
    if (lane < kBlocks) entry = a.page_table[(int64_t)b * a.max_pages + min(j_first + lane, j_last)];
#pragma unroll
    for (int i = 0; i < kBlocks; ++i) {
      const int tb = w_begin + 16 * i;
      const int tc = min(tb, (L - 1) & ~15);
      int64_t phys = __builtin_amdgcn_readlane(entry, (tc >> a.page_shift) - j_first);
      phys = phys < 0 ? 0 : (phys >= a.num_pages ? a.num_pages - 1 : phys);
      brows[i] = min(max(L - tb, 0), 16);
      belem[i] = phys * a.c_page + (int64_t)hk * a.c_head + (int64_t)(tc & pmask) * hd;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kBlocks; ++i) {
      const int tb = w_begin + 16 * i;
      brows[i] = min(max(L - tb, 0), 16);
      belem[i] = (int64_t)b * a.c_seq + (int64_t)hk * a.c_head + (int64_t)min(tb, (L - 1) & ~15) * hd;
    }
  }

#pragma unroll
  for (int i = 0; i < kBlocks; ++i) {  // wave-uniform by construction; keep them in SGPRs
    belem[i] = uniform64(belem[i]);
    brows[i] = __builtin_amdgcn_readfirstlane(brows[i]);
  }

  // q^T as the B operand: column n = query head hk*G + n (zero for n >= G),
  // k step s holding the head_dim values the K fragments hold (zero past hd).
  bf16x8 qf[NDB];
  {
    const uint16_t *q = static_cast<const uint16_t *>(a.q);
    const int64_t qrow = (int64_t)b * a.q_sb + (int64_t)(hk * G + n) * a.q_sh;
#pragma unroll
    for (int s = 0; s < NDB; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (n < G && (!kPad || TR::q_offset(s, g) < hd)) v = *reinterpret_cast<const u32x4 *>(q + qrow + TR::q_offset(s, g));
      qf[s] = __builtin_bit_cast(bf16x8, v);
    }
  }
  bf16x8 ident16[2];
  u32x2 ident8[2];
  make_identity(lane, ident16, ident8);

  WaveState<D, kFP8> st;
#pragma unroll
  for (int c = 0; c < 2 * NDB; ++c) st.o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = kNegInf;
  st.l = 0.f;

  // kTiles 32-token tiles per wave, fully unrolled. While tile i is on the
  // matrix cores, tile i+1's K is in flight to registers and its V to this
  // wave's LDS slots. Tiles past the end of the sequence are not processed.
  constexpr int NU = Tile<D, kFP8>::NU;
  char *vlds = smem_v + wave * Tile<D, kFP8>::kVBytes;
  Tile<D, kFP8> buf[2];
  load_k_block<D, kFP8, kPad>(a, belem[0], brows[0], lane, buf[0].k[0], buf[0].ks[0], buf[0].vs[0]);
  load_k_block<D, kFP8, kPad>(a, belem[1], brows[1], lane, buf[0].k[1], buf[0].ks[1], buf[0].vs[1]);
  __builtin_amdgcn_sched_barrier(0);
  load_v_block_lds<D, kFP8, kPad>(a, belem[0], brows[0], lane, vlds);
  load_v_block_lds<D, kFP8, kPad>(a, belem[1], brows[1], lane, vlds + NU * 1024);
  // Vector-memory issue order, pinned with scheduling barriers so that the
  // explicit vmcnt waits below count exactly:
  //   prologue: K(0), V(0);  iteration i: K(i+1) | QK, softmax | wait V(i),
  //   read V(i) from LDS | V(i+1) | PV.
  // Loads retire in issue order, so V(i) has landed once at most |K(i+1)|
  // loads are outstanding.
  constexpr int kKLoads = 2 * NU + (kFP8 ? 4 : 0);  // per tile: K fragments (+ K, V scales)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int it = 0; it < kTiles; ++it) {
    const int t0 = w_begin + it * kTileTokens;
    if (t0 >= L) break;  // uniform; later tiles are past the end too
    if (it + 1 < kTiles) {
      Tile<D, kFP8> &nx = buf[(it + 1) & 1];
      load_k_block<D, kFP8, kPad>(a, belem[2 * it + 2], brows[2 * it + 2], lane, nx.k[0], nx.ks[0], nx.vs[0]);
      load_k_block<D, kFP8, kPad>(a, belem[2 * it + 3], brows[2 * it + 3], lane, nx.k[1], nx.ks[1], nx.vs[1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    bf16x8 pa_hi, pa_lo;
    qk_softmax<D, kFP8>(a.scale_log2, t0, L, lane, buf[it & 1], qf, st, pa_hi, pa_lo);
    __builtin_amdgcn_sched_barrier(0);
    if (it + 1 < kTiles)
      __builtin_amdgcn_s_waitcnt(vmcnt_only(kKLoads));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    VRegs<D, kFP8> vr;
    read_v<D, kFP8>(vlds, lane, vr);
    // the slots are overwritten only after every lane's read has returned
    __builtin_amdgcn_s_waitcnt(kLgkmcntZero);
    __builtin_amdgcn_sched_barrier(0);
    if (it + 1 < kTiles && t0 + kTileTokens < L) {
      load_v_block_lds<D, kFP8, kPad>(a, belem[2 * it + 2], brows[2 * it + 2], lane, vlds);
      load_v_block_lds<D, kFP8, kPad>(a, belem[2 * it + 3], brows[2 * it + 3], lane, vlds + NU * 1024);
    }
    __builtin_amdgcn_sched_barrier(0);
    pv_tile<D, kFP8>(vr, ident8, pa_hi, pa_lo, st);
  }
  __builtin_amdgcn_s_waitcnt(0);  // no LDS load of this wave is still in flight past the item

  // Merge the 4 wave states of the block in LDS.
  float l = st.l;
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  float *so = smem;
  float *sm = smem + kWavesPerBlock * G * D;
  float *sl = sm + kWavesPerBlock * 16;
  if (g == 0) {
    sm[wave * 16 + n] = st.m;
    sl[wave * 16 + n] = l;
  }
  if (n < G) {  // lane (n + 16g): head n, four consecutive head_dim entries per block
#pragma unroll
    for (int c = 0; c < 2 * NDB; ++c)
      *reinterpret_cast<f32x4 *>(so + (wave * G + n) * D + o_col_d<kFP8>(c, 4 * g)) = st.o[c];
  }
  __syncthreads();
  const int64_t item = ((int64_t)b * a.hkv + hk) * a.max_splits + split;
  for (int idx = threadIdx.x; idx < G * D; idx += kBlockThreads) {
    const int head = idx / D;
    const int d = idx - head * D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) M = fmaxf(M, sm[w * 16 + head]);
    float acc = 0.f, lsum = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
      const float e = __builtin_amdgcn_exp2f(sm[w * 16 + head] - M);
      acc += e * so[(w * G + head) * D + d];
      lsum += e * sl[w * 16 + head];
    }
    a.ws_o[(item * G + head) * D + d] = acc;
    if (d == 0) {
      a.ws_ml[(item * G + head) * 2 + 0] = M;
      a.ws_ml[(item * G + head) * 2 + 1] = lsum;
    }
  }
}


// Block-wide exclusive prefix sum of the per-sequence split counts into LDS:
// prefix[b] = sum_{b' < b} n(L_b'), prefix[B] = total, with n(L) = ceil(L /
// split) + extra for L > 0 (0 for L = 0); lens[b] = L_b (when lens is not null).
__device__ __forceinline__ int split_count(int L, int split_tokens, int extra) {
  return L > 0 ? (L + split_tokens - 1) / split_tokens + extra : 0;
}

__device__ __forceinline__ void build_split_prefix(const DecodeArgs &a, int split_tokens, int *lens, int *prefix,
                                                   int *wave_sums, int extra = 0) {
  const int B = a.batch;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int per = (B + kBlockThreads - 1) / kBlockThreads;
  const int first = tid * per;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    const int b = first + i;
    if (b < B) {
      const int L = max(min(a.seq_lens[b] + a.len_add, a.max_len), 0);
      if (lens != nullptr) lens[b] = L;
      local += split_count(L, split_tokens, extra);
    }
  }
  int v = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  if (lane == 63) wave_sums[wave] = v;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wave_sums[w];
  int run = base + v - local;
  for (int i = 0; i < per; ++i) {
    const int b = first + i;
    if (b < B) {
      prefix[b] = run;
      const int L = lens != nullptr ? lens[b] : max(min(a.seq_lens[b] + a.len_add, a.max_len), 0);
      run += split_count(L, split_tokens, extra);
    }
  }
  if (tid == kBlockThreads - 1) prefix[B] = base + v;
  __syncthreads();
}

// Persistent split kernel: a grid of resident workgroups walks the dense list
// of (sequence, split, KV head) items -- KV heads fastest, so workgroups that
// run together read the head blocks of the same physical pages -- with no
// workgroups for splits past a sequence's end.
template <int D, bool kFP8, int kTiles, bool kPad>
__global__ __launch_bounds__(256, 2) void decode_split_kernel(DecodeArgs a) {
  constexpr int kSplit = kWavesPerBlock * kTiles * kTileTokens;
  constexpr int kVAll = kWavesPerBlock * Tile<D, kFP8>::kVBytes;
  extern __shared__ float smem[];  // V slots [4 waves] | merge area | wave sums | lens[B] | prefix[B + 1]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  char *smem_v = reinterpret_cast<char *>(smem);
  float *merge = reinterpret_cast<float *>(smem_v + kVAll);
  // V slots start at zero: rows past a sequence's end are never written, so
  // what P = 0 meets there is a previous tile's finite V or zero.
  for (int i = threadIdx.x; i < kVAll / 16; i += kBlockThreads)
    reinterpret_cast<u32x4 *>(smem_v)[i] = u32x4{0u, 0u, 0u, 0u};
  int *wave_sums = reinterpret_cast<int *>(merge + merge_floats(a.group, D));
  int *lens = wave_sums + kWavesPerBlock;
  int *prefix = lens + a.batch;
  build_split_prefix(a, kSplit, lens, prefix, wave_sums);
  const int total = __builtin_amdgcn_readfirstlane(prefix[a.batch]) * a.hkv;
  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int hk = item % a.hkv;
    const int sidx = item / a.hkv;
    int lo = 0, hi = a.batch;  // largest b with prefix[b] <= sidx
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (prefix[mid] <= sidx) lo = mid; else hi = mid;
    }
    const int b = __builtin_amdgcn_readfirstlane(lo);
    const int split = sidx - __builtin_amdgcn_readfirstlane(prefix[b]);
    const int L = __builtin_amdgcn_readfirstlane(lens[b]);
    split_item<D, kFP8, kTiles, kPad>(a, b, hk, split, L, lane, wave, smem_v, merge);
    __syncthreads();  // the merge area is reused by the next item
  }
}

// ---------------------------------------------------------------------------
// Balanced partition ("stream-K" over tiles). The work is the flat list of
// 32-token tiles of every (sequence, KV head) segment, segments in (b, hk)
// order, KV heads fastest: W = H_kv * sum_b ceil(L_b / 32) tiles. Wave w of
// the NW resident waves takes tiles [w W / NW, (w + 1) W / NW), so every wave
// streams the same number of bytes (within one tile) whatever the length
// mix, and waves never wait for each other. The piece of a segment that wave
// w holds goes to workspace slot (segment index + w) -- injective, because
// walking the line of tiles, each piece boundary advances the segment, the
// wave, or both -- and a second kernel merges each segment's pieces. (Merging
// in the kernel itself, by the last wave to finish a segment, needs an
// agent-scope release per piece -- an L2 write-back on every arrival -- and
// measured slower than the second launch.)

// Tile range start of wave w.
__host__ __device__ __forceinline__ int64_t wave_first_tile(int64_t w, int64_t W, int64_t NW) { return w * W / NW; }
// The wave whose range holds tile t (the largest w with wave_first_tile(w) <= t).
__host__ __device__ __forceinline__ int64_t wave_of_tile(int64_t t, int64_t W, int64_t NW) {
  return ((t + 1) * NW - 1) / W;
}

// Merge the pieces of segment (b, hk) held by waves w0..w1 (waves with empty
// ranges hold none) and write its G output rows:
// out = sum_p 2^(m_p - M) o_p / sum_p 2^(m_p - M) l_p.
// Up to 64 pieces at a time: lane k loads piece k's maxima and sums for every
// head (one vector load each), the batch maximum and weighted sum come from
// wave reductions, and the partial rows are summed with lane = head_dim
// column, kBatch pieces' loads ahead of their adds. The first row batch is
// loaded together with the maxima and sums, so a segment of up to kBatch
// pieces costs one memory round trip after the prefix.
template <int D, int kMaxG>
__device__ __forceinline__ void merge_segment(const DecodeArgs &a, int b, int hk, int64_t seg, int64_t w0, int64_t w1,
                                              int64_t W, int64_t NW, int lane) {
  constexpr int DPL = D >= 64 ? D / 64 : 1;  // columns lane + 64 j of the D-wide partial rows
  const bool lane_in = D >= 64 || lane < D;
  constexpr int kBatch = 64 / (kMaxG * DPL) < 2 ? 2 : (64 / (kMaxG * DPL) > 16 ? 16 : 64 / (kMaxG * DPL));
  const int G = a.group;  // <= kMaxG
  float M[kMaxG], Ls[kMaxG], acc[kMaxG][DPL];
#pragma unroll
  for (int h = 0; h < kMaxG; ++h) {
    M[h] = kNegInf;
    Ls[h] = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[h][j] = 0.f;
  }
  // With W >= NW every wave holds at least one tile, so every wave of w0..w1
  // holds a piece; only otherwise is a wave's range tested (64-bit divisions).
  const bool every_wave = W >= NW;
  for (int64_t wb = w0; wb <= w1; wb += 64) {
    const int64_t w = wb + lane;
    const bool valid = w <= w1 && (every_wave || wave_first_tile(w, W, NW) < wave_first_tile(w + 1, W, NW));
    const int slot_rel = (int)(valid ? w - w0 : 0);  // slot = seg + w0 + slot_rel; slot w0 always holds a piece
    const int nk = (int)(w1 - wb + 1 < 64 ? w1 - wb + 1 : 64);
    float ov[kBatch][kMaxG][DPL];
    auto load_rows = [&](int k0) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (k0 + u >= nk) break;  // uniform: rows past the batch's pieces are neither loaded nor added
        const int k = k0 + u;
        const int64_t sk = seg + w0 + __builtin_amdgcn_readlane(slot_rel, k);
#pragma unroll
        for (int h = 0; h < kMaxG; ++h)
          if (h < G)
#pragma unroll
            for (int j = 0; j < DPL; ++j) ov[u][h][j] = lane_in ? a.ws_o[(sk * G + h) * D + lane + 64 * j] : 0.f;
      }
    };
    load_rows(0);
    const int64_t slot = seg + w0 + slot_rel;
    float e[kMaxG];
#pragma unroll
    for (int h = 0; h < kMaxG; ++h) {
      e[h] = 0.f;
      if (h < G) {
        const float m = valid ? a.ws_ml[(slot * G + h) * 2] : kNegInf;
        const float l = a.ws_ml[(slot * G + h) * 2 + 1];
        const float m_new = fmaxf(M[h], wave_max(m));  // finite: wave w0 holds a piece
        const float sc = __builtin_amdgcn_exp2f(M[h] - m_new);
        e[h] = valid ? __builtin_amdgcn_exp2f(m - m_new) : 0.f;
        Ls[h] = Ls[h] * sc + wave_sum(valid ? e[h] * l : 0.f);
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[h][j] *= sc;
        M[h] = m_new;
      }
    }
    for (int k0 = 0; k0 < nk; k0 += kBatch) {
      if (k0 > 0) load_rows(k0);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (k0 + u < nk) {  // uniform
#pragma unroll
          for (int h = 0; h < kMaxG; ++h) {
            if (h < G) {
              const float ek = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e[h]), k0 + u));
#pragma unroll
              for (int j = 0; j < DPL; ++j) acc[h][j] += ek * ov[u][h][j];
            }
          }
        }
      }
    }
  }
  uint16_t *out = static_cast<uint16_t *>(a.out) + (int64_t)b * a.o_sb + (int64_t)hk * G * a.o_sh;
#pragma unroll
  for (int h = 0; h < kMaxG; ++h) {
    if (h < G) {
      const float inv = Ls[h] > 0.f ? 1.0f / Ls[h] : 0.f;
#pragma unroll
      for (int j = 0; j < DPL; ++j)
        if (lane + 64 * j < a.head_dim) out[(int64_t)h * a.o_sh + lane + 64 * j] = f32_to_bf16_bits(acc[h][j] * inv);
    }
  }
}

// ---- fused RoPE + append (decode_stream_append_kernel) ----------------------

// Element i of a q / k / v input row: the bf16 activation, or (kPartIn) the
// bf16 sum of the split-K partials added in order (the projection's rounded
// output). Branch-free, so the prologue's loads all go out before any wait:
// kMaxApSplits loads (indices clamped in bounds; at most that many splits,
// checked by the host) before the first add.

template <bool kPartIn>
struct ApRaw {
  float v[kPartIn ? kMaxApSplits : 1];  // the splits, or the bf16 bits (low half) of the activation
};

template <bool kPartIn>
__device__ __forceinline__ void ap_load(const DecodeAppend &ap, const void *p, int64_t i, ApRaw<kPartIn> &r) {
  if constexpr (kPartIn) {
    const float *f = static_cast<const float *>(p);
    const int S = ap.part_splits;
#pragma unroll
    for (int s = 0; s < kMaxApSplits; ++s) r.v[s] = f[(int64_t)(s < S ? s : S - 1) * ap.part_stride + i];
  } else {
    r.v[0] = __uint_as_float((uint32_t)static_cast<const uint16_t *>(p)[i]);
  }
}

template <bool kPartIn>
__device__ __forceinline__ float ap_value(const DecodeAppend &ap, const ApRaw<kPartIn> &r) {
  if constexpr (kPartIn) {
    float acc = r.v[0];
#pragma unroll
    for (int s = 1; s < kMaxApSplits; ++s) acc = s < ap.part_splits ? acc + r.v[s] : acc;
    return round_bf16(acc);
  } else {
    return __uint_as_float(__float_as_uint(r.v[0]) << 16);
  }
}

// Start of a piece of the fused kernel, issued together with the piece's
// first page-table load so that all of it costs one memory round trip (the
// loads are unconditional, with clamped in-bounds addresses, so no wait is
// forced between them):
//  - with `append` (the piece holds its segment's last tile, which only this
//    wave reads): RoPE of this step's k for (b, hk) at position pos and the
//    append of k and v to the cache slot, with the arithmetic of
//    rope_append_kernel (lane i < D/2 owns the pair (i, i + D/2)); skipped
//    when the slot is outside the cache or the table, as that kernel skips it;
//  - RoPE of the G query rows of (b, hk) into the wave's LDS staging area qs
//    [G][D] (bf16), then the MFMA B fragments from it.
template <int D, bool kFP8, bool kPartIn, bool kPad>
__device__ __forceinline__ void piece_prologue(const DecodeArgs &a, const DecodeAppend &ap, int b, int hk, int pos,
                                               bool append, int lane, uint16_t *qs, bf16x8 (&qf)[D / 32]) {
  const int hd = row_len<D, kPad>(a);
  const int H = hd / 2;   // rotation pairs (i, i + H) of a row
  constexpr int kIt = 4;  // query pairs per lane per round (one round for G * D <= 512)
  const int G = a.group;
  const int pairs = G * H;
  const bool in_table = pos >= 0 && pos < ap.table_len;
  const int tp = pos < 0 ? 0 : (pos >= ap.table_len ? (int)ap.table_len - 1 : pos);  // in bounds
  const uint16_t *tab = static_cast<const uint16_t *>(ap.table) + (int64_t)tp * hd;
  const bool active = lane < H;
  const int li = active ? lane : 0;  // lanes past H load pair 0 and drop it

  // loads: append inputs and slot (always, in bounds), then the query inputs;
  // all issued before the scheduling barrier, consumed after it
  const int64_t ks = (int64_t)b * ap.ki_sb + (int64_t)hk * ap.ki_sh;
  const int64_t vs = (int64_t)b * ap.vi_sb + (int64_t)hk * ap.vi_sh;
  ApRaw<kPartIn> kr[4];
  ap_load<kPartIn>(ap, ap.k_in, ks + li, kr[0]);
  ap_load<kPartIn>(ap, ap.k_in, ks + H + li, kr[1]);
  ap_load<kPartIn>(ap, ap.v_in, vs + li, kr[2]);
  ap_load<kPartIn>(ap, ap.v_in, vs + H + li, kr[3]);
  const uint32_t kc_raw = tab[li];
  const uint32_t ks_raw = tab[H + li];
  const int64_t jp = pos < 0 ? 0 : (int64_t)pos >> a.page_shift;
  int64_t phys = 0;
  if (a.page_table != nullptr)
    phys = a.page_table[(int64_t)b * a.max_pages + (jp < a.max_pages ? jp : a.max_pages - 1)];
  ApRaw<kPartIn> qr[kIt][2];
  uint32_t c_raw[kIt], s_raw[kIt];
  auto load_q = [&](int p0) {
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int pr0 = p0 + lane + 64 * it;
      const int pr = pr0 < pairs ? pr0 : pairs - 1;
      const int h = pr / H;
      const int i = pr - h * H;
      const int64_t src = (int64_t)b * ap.qi_sb + (int64_t)(hk * G + h) * ap.qi_sh;
      ap_load<kPartIn>(ap, ap.q_in, src + i, qr[it][0]);
      ap_load<kPartIn>(ap, ap.q_in, src + H + i, qr[it][1]);
      c_raw[it] = tab[i];
      s_raw[it] = tab[H + i];
    }
  };
  auto rope_q = [&](int p0) {
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int pr = p0 + lane + 64 * it;
      if (pr < pairs) {
        const int h = pr / H;
        const int i = pr - h * H;
        float o1, o2;
        rotate_pair<BF16Tag>(ap_value<kPartIn>(ap, qr[it][0]), ap_value<kPartIn>(ap, qr[it][1]),
                             bf16_bits_to_f32((uint16_t)c_raw[it]), bf16_bits_to_f32((uint16_t)s_raw[it]), o1, o2);
        qs[h * D + i] = f32_to_bf16_bits(o1);
        qs[h * D + H + i] = f32_to_bf16_bits(o2);
      }
    }
  };
  load_q(0);
  __builtin_amdgcn_sched_barrier(0);
  const float k1x = ap_value<kPartIn>(ap, kr[0]);
  const float k2x = ap_value<kPartIn>(ap, kr[1]);
  const float v1 = ap_value<kPartIn>(ap, kr[2]);
  const float v2 = ap_value<kPartIn>(ap, kr[3]);
  const float kc = bf16_bits_to_f32((uint16_t)kc_raw);
  const float ksn = bf16_bits_to_f32((uint16_t)ks_raw);

  const bool do_append = append && in_table && pos < ap.capacity;
  // the append
  if (do_append) {
    int64_t base = -1;
    if (a.page_table != nullptr) {
      phys = __builtin_amdgcn_readfirstlane((int)phys);
      if (jp < a.max_pages && phys >= 0 && phys < a.num_pages)
        base = phys * a.c_page + (int64_t)(pos - ((pos >> a.page_shift) << a.page_shift)) * hd;
    } else {
      const int64_t j = pos / ap.page_size;
      base = (int64_t)b * a.c_seq + j * a.c_page + (pos - j * ap.page_size) * hd;
    }
    if (base >= 0) {
      const int64_t off = base + (int64_t)hk * a.c_head;
      float k1 = 0.f, k2 = 0.f;
      if (active) rotate_pair<BF16Tag>(k1x, k2x, kc, ksn, k1, k2);
      if constexpr (!kFP8) {
        uint16_t *kcache = static_cast<uint16_t *>(const_cast<void *>(a.k_cache));
        uint16_t *vcache = static_cast<uint16_t *>(const_cast<void *>(a.v_cache));
        if (active) {
          kcache[off + lane] = f32_to_bf16_bits(k1);
          kcache[off + H + lane] = f32_to_bf16_bits(k2);
          vcache[off + lane] = f32_to_bf16_bits(v1);
          vcache[off + H + lane] = f32_to_bf16_bits(v2);
        }
      } else {
        // per-(token, head) symmetric scale: absmax / 448, codes e4m3fn(x / scale)
        const float kscale = wave_max_nan(absmax2(0.f, k1, k2)) / 448.0f;
        const float vscale = wave_max_nan(absmax2(0.f, v1, v2)) / 448.0f;
        uint8_t *kcache = static_cast<uint8_t *>(const_cast<void *>(a.k_cache));
        uint8_t *vcache = static_cast<uint8_t *>(const_cast<void *>(a.v_cache));
        if (active) {
          kcache[off + lane] = e4m3_row_code(k1, kscale);
          kcache[off + H + lane] = e4m3_row_code(k2, kscale);
          vcache[off + lane] = e4m3_row_code(v1, vscale);
          vcache[off + H + lane] = e4m3_row_code(v2, vscale);
        }
        if (lane == 0) {
          const int64_t sidx = fp8_scale_index(scale_row<D, kPad>(a, off));
          const_cast<float *>(a.k_scale)[sidx] = kscale;
          const_cast<float *>(a.v_scale)[sidx] = vscale;
        }
      }
    }
  }

  // the query rows (further rounds only for G * D > 512)
  rope_q(0);
  for (int p0 = 64 * kIt; p0 < pairs; p0 += 64 * kIt) {
    load_q(p0);
    __builtin_amdgcn_sched_barrier(0);
    rope_q(p0);
  }
  __builtin_amdgcn_s_waitcnt(kLgkmcntZero);
  __builtin_amdgcn_wave_barrier();
  using TR = KVTraits<kFP8>;
  const int n = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int s = 0; s < D / 32; ++s) {
    u32x4 v = {0u, 0u, 0u, 0u};
    // staging entries past hd were never written: zero (query values past head_dim)
    if (n < G && (!kPad || TR::q_offset(s, g) < hd)) v = *reinterpret_cast<const u32x4 *>(qs + n * D + TR::q_offset(s, g));
    qf[s] = __builtin_bit_cast(bf16x8, v);
  }
  __builtin_amdgcn_s_waitcnt(kLgkmcntZero);
  __builtin_amdgcn_wave_barrier();
}

// Tiles [j0, j1) of segment (b, hk) (L tokens) by this wave: the online-softmax
// state over them (unnormalised O, the heads' maxima, lane-partial sums) in st.
template <int D, bool kFP8, bool kAppend, bool kPartIn, bool kPad>
__device__ __forceinline__ void stream_piece(const DecodeArgs &a, const DecodeAppend *ap, int b, int hk, int L,
                                             int j0, int j1, bool append, int lane, char *vlds, uint16_t *qs,
                                             const bf16x8 (&ident16)[2], const u32x2 (&ident8)[2],
                                             WaveState<D, kFP8> &st) {
  using TR = KVTraits<kFP8>;
  constexpr int NDB = D / 32;
  const int G = a.group;
  const int n = lane & 15;
  const int g = lane >> 4;

  bf16x8 qf[NDB];
  int entry0 = 0;
  if constexpr (kAppend) {
    // the first chunk's page entries go out with the prologue's loads
    if (a.page_table != nullptr) {
      const int pb0 = (kTileTokens * j0) >> a.page_shift;
      entry0 = a.page_table[(int64_t)b * a.max_pages + min(pb0 + lane, (L - 1) >> a.page_shift)];
    }
    piece_prologue<D, kFP8, kPartIn, kPad>(a, *ap, b, hk, __builtin_amdgcn_readfirstlane(a.seq_lens[b]), append, lane,
                                           qs, qf);
    // The appended token is in this piece's last tile. Its loads are issued
    // after the tile loop's first explicit vmcnt wait (which retires the
    // stores above) unless it is one of the first chunk's first two tiles.
    if (append && j1 - j0 <= 2) __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
  } else {
    const uint16_t *q = static_cast<const uint16_t *>(a.q);
    const int64_t qrow = (int64_t)b * a.q_sb + (int64_t)(hk * G + n) * a.q_sh;
    const int hd = row_len<D, kPad>(a);
#pragma unroll
    for (int s = 0; s < NDB; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (n < G && (!kPad || TR::q_offset(s, g) < hd)) v = *reinterpret_cast<const u32x4 *>(q + qrow + TR::q_offset(s, g));
      qf[s] = __builtin_bit_cast(bf16x8, v);
    }
  }
#pragma unroll
  for (int c = 0; c < 2 * NDB; ++c) st.o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = kNegInf;
  st.l = 0.f;

  constexpr int NU = Tile<D, kFP8>::NU;
  constexpr int kKLoads = 2 * NU + (kFP8 ? 4 : 0);  // per tile: K fragments (+ K, V scales)
  // Chunks of kChunkTiles tiles, each fully unrolled so the two K buffers
  // alternate with static indices. Vector-memory issue order, pinned with
  // scheduling barriers so that the explicit vmcnt waits count exactly:
  //   chunk start: page entries, K(0), V(0);  tile k: K(k+1) | QK, softmax |
  //   wait V(k), read V(k) from LDS | V(k+1) | PV.
  // Loads retire in issue order, so V(k) has landed once at most |K(k+1)|
  // loads are outstanding. K(k+1) is issued for every k + 1 < kChunkTiles
  // (rows past the end read nothing), so no buffer is conditionally written.
  for (int c0 = j0; c0 < j1; c0 += kChunkTiles) {
    const int c1 = min(j1, c0 + kChunkTiles);
    int entry = 0, pbase = 0;
    if (a.page_table != nullptr) {
      pbase = (kTileTokens * c0) >> a.page_shift;
      const int last = (L - 1) >> a.page_shift;
      entry = (kAppend && c0 == j0) ? entry0 : a.page_table[(int64_t)b * a.max_pages + min(pbase + lane, last)];
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
    for (int k = 0; k < kChunkTiles; ++k) {
      const int it = c0 + k;
      if (it >= c1) break;  // uniform
      if (k + 1 < kChunkTiles) {
        stream_block_addr<D, kPad>(a, b, hk, L, entry, pbase, 2 * it + 2, e0, r0);
        stream_block_addr<D, kPad>(a, b, hk, L, entry, pbase, 2 * it + 3, e1, r1);
        Tile<D, kFP8> &nx = buf[(k + 1) & 1];
        load_k_block<D, kFP8, kPad>(a, e0, r0, lane, nx.k[0], nx.ks[0], nx.vs[0]);
        load_k_block<D, kFP8, kPad>(a, e1, r1, lane, nx.k[1], nx.ks[1], nx.vs[1]);
      }
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 pa_hi, pa_lo;
      qk_softmax<D, kFP8>(a.scale_log2, kTileTokens * it, L, lane, buf[k & 1], qf, st, pa_hi, pa_lo);
      __builtin_amdgcn_sched_barrier(0);
      if (k + 1 < kChunkTiles)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(kKLoads));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
      VRegs<D, kFP8> vr;
      read_v<D, kFP8>(vlds, lane, vr);
      // the slots are overwritten only after every lane's read has returned
      __builtin_amdgcn_s_waitcnt(kLgkmcntZero);
      __builtin_amdgcn_sched_barrier(0);
      if (k + 1 < kChunkTiles && it + 1 < c1) {
        load_v_block_lds<D, kFP8, kPad>(a, e0, r0, lane, vlds);
        load_v_block_lds<D, kFP8, kPad>(a, e1, r1, lane, vlds + NU * 1024);
      }
      __builtin_amdgcn_sched_barrier(0);
      pv_tile<D, kFP8>(vr, ident8, pa_hi, pa_lo, st);
    }
    __builtin_amdgcn_s_waitcnt(0);  // nothing of this chunk still in flight
  }
}

// A piece's state to workspace slot `slot` (the balanced partition's partials).
template <int D, bool kFP8>
__device__ __forceinline__ void store_piece(const DecodeArgs &a, const WaveState<D, kFP8> &st, int64_t slot,
                                            int lane) {
  constexpr int NDB = D / 32;
  const int G = a.group;
  const int n = lane & 15;
  const int g = lane >> 4;
  float l = st.l;  // lane-partial sums -> the head's sum in all 4 lanes of the head
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (n < G) {  // lane (n + 16g): head n, four consecutive head_dim entries per block (16-byte stores)
#pragma unroll
    for (int c = 0; c < 2 * NDB; ++c)
      *reinterpret_cast<f32x4 *>(a.ws_o + (slot * G + n) * D + o_col_d<kFP8>(c, 4 * g)) = st.o[c];
  }
  if (g == 0 && n < G) {
    a.ws_ml[(slot * G + n) * 2 + 0] = st.m;
    a.ws_ml[(slot * G + n) * 2 + 1] = l;
  }
}

// Persistent balanced kernel: NW = gridDim.x * 4 waves, all resident. The
// code is compiled for kStreamOcc workgroups per CU (register budget) and
// launched with stream_blocks_per_cu(D) of them: at head_dim 128 four
// streaming waves per CU measured best (fewer, longer runs per wave and
// fewer partials; C2 -10 %, C3 -1 % against eight); at head_dim 64 a tile is
// half the bytes, four waves keep too little in flight, and eight measured
// better (C5 step -5 %, end to end +2 %).
constexpr int kStreamOcc = 2;
constexpr int stream_blocks_per_cu(int tile_d) { return tile_d <= 64 ? 2 : 1; }

// Tiles' worth of time a wave spends starting a segment piece (length and
// page-table lookups, q fragments, the fused step's RoPE + append): charged to
// every segment in the balanced partition, so a wave that holds many short
// segments gets fewer tiles. Measured (fused step, 0 -> 2): C3 406 -> 387 us,
// C4 802 -> 766 us, C2 113 -> 110 us, C5 layer 39.3 -> 37.8 us; 1, 3 and 4
// were as good or worse on every config.
constexpr int stream_seg_cost(int /*head_dim*/) { return kStreamSegCost; }

// LDS of the split kernel: V slots [4 waves] | wave sums [4] | prefix [B + 1]
// (| q staging [4 waves][16][D] bf16 for the fused variant).
template <int D, bool kFP8, bool kAppend, bool kPartIn, bool kPad>
__device__ __forceinline__ void stream_body(const DecodeArgs &a, const DecodeAppend *ap) {
  constexpr int kVAll = kWavesPerBlock * Tile<D, kFP8>::kVBytes;
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  char *smem_v = reinterpret_cast<char *>(smem);
  for (int i = threadIdx.x; i < kVAll / 16; i += kBlockThreads)
    reinterpret_cast<u32x4 *>(smem_v)[i] = u32x4{0u, 0u, 0u, 0u};
  int *wave_sums = reinterpret_cast<int *>(smem_v + kVAll);
  int *prefix = wave_sums + kWavesPerBlock;
  uint16_t *qs = nullptr;
  if constexpr (kAppend)
    qs = reinterpret_cast<uint16_t *>(smem_v + kVAll + 16 * ((sizeof(int) * (kWavesPerBlock + a.batch + 1) + 15) / 16)) +
         wave * 16 * D;
  build_split_prefix(a, kTileTokens, nullptr, prefix, wave_sums, a.seg_cost);  // ends with a block barrier
  if (blockIdx.x == 0) {  // for the merge kernel (and the next step's lengths)
    for (int i = threadIdx.x; i <= a.batch; i += kBlockThreads) a.ws_prefix[i] = prefix[i];
    if constexpr (kAppend)
      if (ap->lens_out != nullptr)
        for (int i = threadIdx.x; i < a.batch; i += kBlockThreads) ap->lens_out[i] = a.seq_lens[i] + 1;
  }
  const int64_t W = (int64_t)__builtin_amdgcn_readfirstlane(prefix[a.batch]) * a.hkv;
  const int64_t NW = a.stream_waves;
  const int64_t w = (int64_t)blockIdx.x * kWavesPerBlock + wave;
  int64_t t = uniform64(wave_first_tile(w, W, NW));
  const int64_t t_end = uniform64(wave_first_tile(w + 1, W, NW));
  bf16x8 ident16[2];
  u32x2 ident8[2];
  make_identity(lane, ident16, ident8);
  char *vlds = smem_v + wave * Tile<D, kFP8>::kVBytes;
  while (t < t_end) {
    int lo = 0, hi = a.batch;  // largest b with hkv * prefix[b] <= t
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if ((int64_t)prefix[mid] * a.hkv <= t) lo = mid; else hi = mid;
    }
    const int b = __builtin_amdgcn_readfirstlane(lo);
    const int pb = __builtin_amdgcn_readfirstlane(prefix[b]);
    const int nbe = __builtin_amdgcn_readfirstlane(prefix[b + 1]) - pb;  // > 0: tile t lies in sequence b
    const int64_t local = t - (int64_t)pb * a.hkv;
    const int hk = (int)(local / nbe);
    const int j0e = (int)(local - (int64_t)hk * nbe);
    const int64_t seg_end = (int64_t)pb * a.hkv + (int64_t)(hk + 1) * nbe;
    const int64_t stop = seg_end < t_end ? seg_end : t_end;
    // real tiles of the piece: the segment's first seg_cost line positions hold none
    const int j0 = max(j0e - a.seg_cost, 0);
    const int j1 = j0e + (int)(stop - t) - a.seg_cost;
    if (j1 > j0) {
      const int L = __builtin_amdgcn_readfirstlane(min(a.seq_lens[b] + a.len_add, a.max_len));
      // The segment's last tile holds this step's token: only this wave reads
      // it, so the fused variant appends it at the start of this piece.
      WaveState<D, kFP8> st;
      stream_piece<D, kFP8, kAppend, kPartIn, kPad>(a, ap, b, hk, L, j0, j1, kAppend && j1 == nbe - a.seg_cost, lane,
                                                    vlds, qs, ident16, ident8, st);
      store_piece<D, kFP8>(a, st, (int64_t)b * a.hkv + hk + w, lane);
    }
    t = stop;
  }
}

template <int D, bool kFP8, bool kPad>
__global__ __launch_bounds__(256, kStreamOcc) void decode_stream_kernel(DecodeArgs a) {
  stream_body<D, kFP8, false, false, kPad>(a, nullptr);
}

// The same split kernel with this step's RoPE + append folded in (q rotated
// per piece from the projection outputs; k / v written by the wave that
// reads the segment's last tile).
template <int D, bool kFP8, bool kPartIn, bool kPad>
__global__ __launch_bounds__(256, kStreamOcc) void decode_stream_append_kernel(DecodeAppendArgs a) {
  stream_body<D, kFP8, true, kPartIn, kPad>(a, &a.ap);
}

// LDS of the per-segment kernel: the streaming area (V slots, q staging of
// the fused variant) and the merge area ([4][G][D] + 2 [4][16] floats), side
// by side when that fits in 64 KB, else the merge area over the streaming one.
__host__ __device__ constexpr int segment_stream_lds(int tile_d, bool fp8, bool fused) {
  return kWavesPerBlock * 2 * (tile_d * (fp8 ? 1 : 2) / 64) * 1024 + (fused ? kWavesPerBlock * 16 * tile_d * 2 : 0);
}
__host__ __device__ constexpr int segment_merge_lds(int tile_d, int group) {
  return (int)sizeof(float) * merge_floats(group, tile_d);
}
__host__ __device__ constexpr bool segment_merge_separate(int tile_d, bool fp8, bool fused, int group) {
  return segment_stream_lds(tile_d, fp8, fused) + segment_merge_lds(tile_d, group) <= 65536;
}

// ---------------------------------------------------------------------------
// Per-segment partition (split_tokens == kSplitPerSegment): one workgroup per
// (sequence, KV head) segment, workgroup index = segment index, its 4 waves
// taking the quarters of the segment's line as the balanced partition draws it
// (start-up positions, then the tiles). The 4 wave states merge in LDS and the
// workgroup writes the G
// normalised output rows itself: no workspace and no merge launch. Correct for
// any lengths; balanced when every sequence has the same length and B * H_kv
// fills whole rounds of the resident workgroups (the uniform batches of the
// reference's engine).
// LDS: segment_stream_lds, then (segment_merge_separate) the merge area.
template <int D, bool kFP8, bool kAppend, bool kPartIn, bool kPad>
__device__ __forceinline__ void segment_body(const DecodeArgs &a, const DecodeAppend *ap) {
  constexpr int kVAll = kWavesPerBlock * Tile<D, kFP8>::kVBytes;
  constexpr int NDB = D / 32;
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  char *smem_v = reinterpret_cast<char *>(smem);
  for (int i = threadIdx.x; i < kVAll / 16; i += kBlockThreads)
    reinterpret_cast<u32x4 *>(smem_v)[i] = u32x4{0u, 0u, 0u, 0u};
  uint16_t *qs = nullptr;
  if constexpr (kAppend) {
    qs = reinterpret_cast<uint16_t *>(smem_v + kVAll) + wave * 16 * D;
    if (blockIdx.x == 0 && ap->lens_out != nullptr)  // the next step's lengths
      for (int i = threadIdx.x; i < a.batch; i += kBlockThreads) ap->lens_out[i] = a.seq_lens[i] + 1;
  }
  __syncthreads();  // V slots zeroed

  const int G = a.group;
  const int b = (int)(blockIdx.x / (unsigned)a.hkv);
  const int hk = (int)(blockIdx.x - (unsigned)b * (unsigned)a.hkv);
  const int L = __builtin_amdgcn_readfirstlane(max(min(a.seq_lens[b] + a.len_add, a.max_len), 0));
  const int nt = (L + kTileTokens - 1) / kTileTokens;
  // The quarters of the balanced partition's line for one segment: its
  // kStreamSegCost start-up positions, then the nt tiles. Against quarters of
  // the tiles alone (wave q starting at tile q nt / 4, for C2 at multiples of
  // 256 KB into the segment in every workgroup) the waves streamed ~5 % slower
  // (C2 mean wave end 83-85 against 88-90 us, lab timestamps).
  const int np = nt + kStreamSegCost;
  const int j0 = max(wave * np / kWavesPerBlock - kStreamSegCost, 0);
  const int j1 = max((wave + 1) * np / kWavesPerBlock - kStreamSegCost, 0);
  WaveState<D, kFP8> st;
  if (j1 > j0) {
    bf16x8 ident16[2];
    u32x2 ident8[2];
    make_identity(lane, ident16, ident8);
    // the wave holding the last tile appends this step's token (fused variant)
    stream_piece<D, kFP8, kAppend, kPartIn, kPad>(a, ap, b, hk, L, j0, j1, kAppend && j1 == nt, lane,
                                                  smem_v + wave * Tile<D, kFP8>::kVBytes, qs, ident16, ident8, st);
  } else {
#pragma unroll
    for (int c = 0; c < 2 * NDB; ++c) st.o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = kNegInf;
    st.l = 0.f;
  }
  // The merge area follows the streaming area when both fit in 64 KB, so a
  // wave stores its state as soon as it is done; otherwise it reuses the
  // streaming area once every wave is done with it.
  float *so;  // [4][G][D] unnormalised outputs, then [4][16] maxima and [4][16] sums
  if (segment_merge_separate(D, kFP8, kAppend, G)) {
    so = reinterpret_cast<float *>(smem_v + segment_stream_lds(D, kFP8, kAppend));
  } else {
    __syncthreads();
    so = smem;
  }
  float *sm = so + kWavesPerBlock * G * D;
  float *sl = sm + kWavesPerBlock * 16;
  const int n = lane & 15;
  const int g = lane >> 4;
  float l = st.l;  // lane-partial sums -> the head's sum in all 4 lanes of the head
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (g == 0) {
    sm[wave * 16 + n] = st.m;
    sl[wave * 16 + n] = l;
  }
  if (n < G) {  // lane (n + 16g): head n, four consecutive head_dim entries per block
#pragma unroll
    for (int c = 0; c < 2 * NDB; ++c)
      *reinterpret_cast<f32x4 *>(so + (wave * G + n) * D + o_col_d<kFP8>(c, 4 * g)) = st.o[c];
  }
  __syncthreads();
  // Thread t merges column pairs (2p, 2p + 1) of head p / (D / 2): one set of
  // head weights per pair, and at G * D <= 512 a single pair per thread.
  uint16_t *out = static_cast<uint16_t *>(a.out) + (int64_t)b * a.o_sb + (int64_t)hk * G * a.o_sh;
  for (int pr = threadIdx.x; pr < G * (D / 2); pr += kBlockThreads) {
    const int head = pr / (D / 2);
    const int d = 2 * (pr - head * (D / 2));
    if (d >= a.head_dim) continue;  // head_dim is even: d + 1 < head_dim too
    float mw[kWavesPerBlock];
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
      mw[w] = sm[w * 16 + head];
      M = fmaxf(M, mw[w]);
    }
    float acc0 = 0.f, acc1 = 0.f, lsum = 0.f;
    if (M != kNegInf) {  // a sequence with nothing cached gives zeros
#pragma unroll
      for (int w = 0; w < kWavesPerBlock; ++w) {
        const float e = __builtin_amdgcn_exp2f(mw[w] - M);
        const float *row = so + (w * G + head) * D + d;
        acc0 += e * row[0];
        acc1 += e * row[1];
        lsum += e * sl[w * 16 + head];
      }
    }
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    out[(int64_t)head * a.o_sh + d] = f32_to_bf16_bits(acc0 * inv);
    out[(int64_t)head * a.o_sh + d + 1] = f32_to_bf16_bits(acc1 * inv);
  }
}

template <int D, bool kFP8, bool kPad>
__global__ __launch_bounds__(256, kStreamOcc) void decode_segment_kernel(DecodeArgs a) {
  segment_body<D, kFP8, false, false, kPad>(a, nullptr);
}

template <int D, bool kFP8, bool kPartIn, bool kPad>
__global__ __launch_bounds__(256, kStreamOcc) void decode_segment_append_kernel(DecodeAppendArgs a) {
  segment_body<D, kFP8, true, kPartIn, kPad>(a, &a.ap);
}

// ---------------------------------------------------------------------------
// Paired partition (split_tokens == kSplitPaired), for ragged batches of up to
// kMaxPairedBatch sequences: the sequences ranked by length (longest first,
// ties by index), workgroup (p, hk) takes the segments of KV head hk of the
// sequences ranked p and B - 1 - p (one for the middle rank of an odd batch),
// whose lengths add up to about the same total in every workgroup. Its NWV
// waves split the two segments' line (each segment's start-up positions, then
// its tiles) evenly, as the balanced partition does the whole batch's, so a
// wave holds at most one piece of each segment; the pieces merge in LDS and the
// workgroup writes both segments' rows: one launch, no workspace.
static_assert(kMaxPairedBatch == 256 && kMaxPairedBatch % 16 == 0, "the paired kernel's LDS holds 256 length keys");
typedef int i32x4 __attribute__((ext_vector_type(4)));
// waves per paired workgroup: as many per CU as the balanced kernel at one
// workgroup per CU
constexpr int paired_waves(int tile_d) { return tile_d <= 64 ? 8 : 4; }

// LDS of the paired kernel: the streaming area (NWV V slots, and q staging for
// the fused variant), later the merge area [NWV][G][D] + maxima and sums
// [NWV][16] each, taken by one segment after the other; then the length keys
// and the pair.
__host__ __device__ constexpr int paired_stream_lds(int tile_d, bool fp8, bool fused, int nwv) {
  return nwv * 2 * (tile_d * (fp8 ? 1 : 2) / 64) * 1024 + (fused ? nwv * 16 * tile_d * 2 : 0);
}
__host__ __device__ constexpr int paired_merge_lds(int tile_d, int group, int nwv) {
  return (int)sizeof(float) * (nwv * group * tile_d + 2 * nwv * 16);
}
__host__ __device__ constexpr int paired_lds(int tile_d, bool fp8, bool fused, int group, int nwv) {
  return (paired_stream_lds(tile_d, fp8, fused, nwv) > paired_merge_lds(tile_d, group, nwv)
              ? paired_stream_lds(tile_d, fp8, fused, nwv)
              : paired_merge_lds(tile_d, group, nwv)) +
         (int)sizeof(int) * ((int)kMaxPairedBatch + 2);
}

template <int D, bool kFP8, bool kAppend, bool kPartIn, bool kPad, int NWV>
__device__ __forceinline__ void paired_body(const DecodeArgs &a, const DecodeAppend *ap) {
  constexpr int kVAll = NWV * Tile<D, kFP8>::kVBytes;
  constexpr int NDB = D / 32;
  constexpr int kPairThreads = 64 * NWV;  // the launch's block size (blockDim.x is a load from the dispatch)
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = a.group;
  const int NB = a.batch;
  char *smem_v = reinterpret_cast<char *>(smem);
  int *keys = reinterpret_cast<int *>(smem_v + (paired_lds(D, kFP8, kAppend, G, NWV) -
                                               (int)sizeof(int) * ((int)kMaxPairedBatch + 2)));
  int *pair = keys + kMaxPairedBatch;
  for (int i = threadIdx.x; i < kVAll / 16; i += kPairThreads)
    reinterpret_cast<u32x4 *>(smem_v)[i] = u32x4{0u, 0u, 0u, 0u};
  uint16_t *qs = nullptr;
  if constexpr (kAppend) {
    qs = reinterpret_cast<uint16_t *>(smem_v + kVAll) + wave * 16 * D;
    if (blockIdx.x == 0 && ap->lens_out != nullptr)  // the next step's lengths
      for (int i = threadIdx.x; i < NB; i += kPairThreads) ap->lens_out[i] = a.seq_lens[i] + 1;
  }
  const int p = (int)(blockIdx.x / (unsigned)a.hkv);
  const int hk = (int)(blockIdx.x - (unsigned)p * (unsigned)a.hkv);
  int bA, bB;  // bB = -1: the middle rank of an odd batch, alone
  int LA, LB;
  if (a.order != nullptr) {
    // the caller's length order (indices clamped into the batch): no ranking
    // on the device, whose serial chain (lengths to LDS, two barriers, the
    // ranking) delayed every tile request by ~2.8 us at the C5 layer
    // The lengths go to LDS in the same round trip as the pair's indices (a
    // load of seq_lens[bA] after that of bA would be a second one, cold).
    for (int b = threadIdx.x; b < NB; b += kPairThreads) keys[b] = max(min(a.seq_lens[b] + a.len_add, a.max_len), 0);
    bA = min(max(a.order[p], 0), NB - 1);
    bB = NB - 1 - p != p ? min(max(a.order[NB - 1 - p], 0), NB - 1) : -1;
    __syncthreads();  // V slots zeroed, lengths in place
    LA = keys[bA];
    LB = bB >= 0 ? keys[bB] : 0;
  } else {
    // keys padded with -1 (below every length) to a multiple of 16
    const int nb16 = (NB + 15) & ~15;
    for (int b = threadIdx.x; b < nb16; b += kPairThreads)
      keys[b] = b < NB ? max(min(a.seq_lens[b] + a.len_add, a.max_len), 0) : -1;
    if (threadIdx.x == 0) pair[1] = -1;
    __syncthreads();  // V slots zeroed, keys in place
    // rank r(b) = sequences before b: longer, or as long with a smaller index;
    // 16 keys per step from four broadcast 16-byte LDS reads
    for (int b = threadIdx.x; b < NB; b += kPairThreads) {
      const int kb = keys[b];
      const i32x4 *k4 = reinterpret_cast<const i32x4 *>(keys);
      int r = 0;
      for (int c0 = 0; c0 < nb16; c0 += 16) {
        i32x4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = k4[c0 / 4 + i];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) r += (v[i][e] > kb || (v[i][e] == kb && c0 + 4 * i + e < b)) ? 1 : 0;
      }
      if (r == p) pair[0] = b;
      if (r == NB - 1 - p && r != p) pair[1] = b;
    }
    __syncthreads();
    bA = pair[0];
    bB = pair[1];
    LA = keys[bA];
    LB = bB >= 0 ? keys[bB] : 0;
  }
  bA = __builtin_amdgcn_readfirstlane(bA);
  bB = __builtin_amdgcn_readfirstlane(bB);
  LA = __builtin_amdgcn_readfirstlane(LA);
  LB = __builtin_amdgcn_readfirstlane(LB);
  const int ntA = (LA + kTileTokens - 1) / kTileTokens;
  const int ntB = (LB + kTileTokens - 1) / kTileTokens;
  const int lineA = ntA > 0 ? ntA + kStreamSegCost : 0;
  const int lineB = ntB > 0 ? ntB + kStreamSegCost : 0;
  const int W = lineA + lineB;
  const int s0 = wave * W / NWV;
  const int s1 = (wave + 1) * W / NWV;

  WaveState<D, kFP8> stA, st;
#pragma unroll
  for (int c = 0; c < 2 * NDB; ++c) stA.o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  stA.m = kNegInf;
  stA.l = 0.f;
  bf16x8 ident16[2];
  u32x2 ident8[2];
  make_identity(lane, ident16, ident8);
  for (int sg = 0; sg < 2; ++sg) {  // this wave's piece of segment A, then of segment B
    const int base = sg == 0 ? 0 : lineA;
    const int line = sg == 0 ? lineA : lineB;
    const int nt = sg == 0 ? ntA : ntB;
    const int b = sg == 0 ? bA : bB;
    const int L = sg == 0 ? LA : LB;
    const int j0 = max(max(s0 - base, 0) - kStreamSegCost, 0);
    const int j1 = max(min(s1 - base, line) - kStreamSegCost, 0);
#pragma unroll
    for (int c = 0; c < 2 * NDB; ++c) st.o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = kNegInf;
    st.l = 0.f;
    if (j1 > j0)  // the wave holding a segment's last tile appends its token (fused variant)
      stream_piece<D, kFP8, kAppend, kPartIn, kPad>(a, ap, b, hk, L, j0, j1, kAppend && j1 == nt, lane,
                                                    smem_v + wave * Tile<D, kFP8>::kVBytes, qs, ident16, ident8, st);
    if (sg == 0) stA = st;
  }
  // The two segments merge one after the other in the same LDS area (over the
  // streaming one): [NWV][G][D] unnormalised outputs, [NWV][16] maxima, sums.
  float *so = smem;
  float *sm = so + NWV * G * D;
  float *sl = sm + NWV * 16;
  const int n = lane & 15;
  const int g = lane >> 4;
  for (int sg = 0; sg < 2; ++sg) {
    const int b = sg == 0 ? bA : bB;
    if (b < 0) break;  // the middle rank of an odd batch: no second segment
    __syncthreads();   // every wave is done with its V slot and q staging, or with the last merge
    const WaveState<D, kFP8> &x = sg == 0 ? stA : st;
    float l = x.l;  // lane-partial sums -> the head's sum in all 4 lanes of the head
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (g == 0) {
      sm[wave * 16 + n] = x.m;
      sl[wave * 16 + n] = l;
    }
    if (n < G) {
#pragma unroll
      for (int c = 0; c < 2 * NDB; ++c)
        *reinterpret_cast<f32x4 *>(so + (wave * G + n) * D + o_col_d<kFP8>(c, 4 * g)) = x.o[c];
    }
    __syncthreads();
    // column pairs (2p, 2p + 1) of every head
    uint16_t *out = static_cast<uint16_t *>(a.out) + (int64_t)b * a.o_sb + (int64_t)hk * G * a.o_sh;
    for (int pr = threadIdx.x; pr < G * (D / 2); pr += kPairThreads) {
      const int head = pr / (D / 2);
      const int d = 2 * (pr - head * (D / 2));
      if (d >= a.head_dim) continue;  // head_dim is even: d + 1 < head_dim too
      float mw[NWV];
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < NWV; ++w) {
        mw[w] = sm[w * 16 + head];
        M = fmaxf(M, mw[w]);
      }
      float acc0 = 0.f, acc1 = 0.f, lsum = 0.f;
      if (M != kNegInf) {  // a sequence with nothing cached gives zeros
#pragma unroll
        for (int w = 0; w < NWV; ++w) {
          const float e = __builtin_amdgcn_exp2f(mw[w] - M);
          const float *row = so + (w * G + head) * D + d;
          acc0 += e * row[0];
          acc1 += e * row[1];
          lsum += e * sl[w * 16 + head];
        }
      }
      const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
      out[(int64_t)head * a.o_sh + d] = f32_to_bf16_bits(acc0 * inv);
      out[(int64_t)head * a.o_sh + d + 1] = f32_to_bf16_bits(acc1 * inv);
    }
  }
}

template <int D, bool kFP8, bool kPad, int NWV>
__global__ __launch_bounds__(64 * NWV, NWV == 4 ? kStreamOcc : 1) void decode_paired_kernel(DecodeArgs a) {
  paired_body<D, kFP8, false, false, kPad, NWV>(a, nullptr);
}

template <int D, bool kFP8, bool kPartIn, bool kPad, int NWV>
__global__ __launch_bounds__(64 * NWV, NWV == 4 ? kStreamOcc : 1) void decode_paired_append_kernel(DecodeAppendArgs a) {
  paired_body<D, kFP8, true, kPartIn, kPad, NWV>(a, &a.ap);
}

// One wave per segment (b, KV head): merge its pieces into the G output rows
// (zeros for a sequence with nothing cached). kMaxG bounds the group size.
template <int D, int kMaxG>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeArgs a) {
  constexpr int DPL = D >= 64 ? D / 64 : 1;
  const int64_t seg = blockIdx.x;
  const int b = (int)(seg / a.hkv);
  const int hk = (int)(seg - (int64_t)b * a.hkv);
  const int lane = threadIdx.x;
  const int pb = a.ws_prefix[b];
  const int nb = a.ws_prefix[b + 1] - pb;
  if (nb <= 0) {
    uint16_t *out = static_cast<uint16_t *>(a.out) + (int64_t)b * a.o_sb + (int64_t)hk * a.group * a.o_sh;
    for (int h = 0; h < a.group; ++h)
      for (int j = 0; j < DPL; ++j)
        if (lane + 64 * j < a.head_dim) out[(int64_t)h * a.o_sh + lane + 64 * j] = 0;
    return;
  }
  const int64_t W = (int64_t)a.ws_prefix[a.batch] * a.hkv;
  const int64_t NW = a.stream_waves;
  // the segment's real tiles sit after its seg_cost empty line positions; every
  // wave whose range meets them holds a piece
  const int64_t start = (int64_t)pb * a.hkv + (int64_t)hk * nb + a.seg_cost;
  const int64_t last = (int64_t)pb * a.hkv + (int64_t)(hk + 1) * nb - 1;
  merge_segment<D, kMaxG>(a, b, hk, seg, wave_of_tile(start, W, NW), wave_of_tile(last, W, NW), W, NW, lane);
}

// VALU path: fp32 caches (small models run in fp32, e.g. the reference
// without autocast) and head dims the MFMA tiles do not take (not a multiple
// of 16 bytes: of 8 bf16 or 16 fp8 values), any even head_dim <= 128. Fixed
// splits, the same workspace contract as the MFMA split kernel (partial rows
// D_ws = ws_d floats wide). Each wave walks its tokens 64 at a time with one
// token per lane for the scores, then one head_dim entry per lane (two past
// 64) for P.V. K/V values: fp32, bf16, or fp8-e4m3 codes times the row scale.
template <CacheKind K>
__device__ __forceinline__ float kv_value(const void *base, int64_t i) {
  if constexpr (K == CacheKind::kF32) {
    return static_cast<const float *>(base)[i];
  } else if constexpr (K == CacheKind::kBF16) {
    return bf16_bits_to_f32(static_cast<const uint16_t *>(base)[i]);
  } else {
    const uint32_t code = static_cast<const uint8_t *>(base)[i];
    return (float)__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(code, 1.0f, false)[0];  // exact
  }
}

template <CacheKind K>
__global__ __launch_bounds__(256) void decode_split_kernel_valu(DecodeArgs a, int ws_d) {
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int split = blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int G = a.group;
  const int hd = a.head_dim;
  const int L = min(a.seq_lens[b], a.max_len);
  const int s_begin = split * a.split_tokens;
  if (s_begin >= L) return;
  // the sequence whose cache row b attends to
  const int bs = a.seq_of_row == nullptr ? b : min(max(a.seq_of_row[b], 0), a.num_seqs - 1);
  const int s_end = min(L, s_begin + a.split_tokens);
  const int per_wave = a.split_tokens / kWavesPerBlock;
  const int w_begin = s_begin + wave * per_wave;
  const int w_end = min(s_end, w_begin + per_wave);

  float *so = smem;                                  // [4][G][ws_d]
  float *sm = so + kWavesPerBlock * G * ws_d;        // [4][16]
  float *sl = sm + kWavesPerBlock * 16;              // [4][16]
  float *sq = sl + kWavesPerBlock * 16;              // [G][hd] query rows
  float *sp = sq + G * hd + wave * 64;               // per-wave [64] probabilities
  for (int idx = threadIdx.x; idx < G * hd; idx += kBlockThreads) {
    const int h = idx / hd;
    const int64_t qi = (int64_t)b * a.q_sb + (int64_t)(hk * G + h) * a.q_sh + (idx - h * hd);
    sq[idx] = K == CacheKind::kF32 ? static_cast<const float *>(a.q)[qi]
                                   : bf16_bits_to_f32(static_cast<const uint16_t *>(a.q)[qi]);
  }
  __syncthreads();

  float o[16][2];
  float mrun[16], lrun[16];
  for (int h = 0; h < 16; ++h) {
    mrun[h] = kNegInf;
    lrun[h] = 0.f;
    o[h][0] = o[h][1] = 0.f;
  }
  for (int t0 = w_begin; t0 < w_end; t0 += 64) {
    const int tok = t0 + lane;
    const bool valid = tok < w_end;
    int64_t koff = 0;
    float ksc = 1.f;
    if (valid) {
      koff = token_elem(a, bs, hk, tok, hd);
      if constexpr (K == CacheKind::kFP8) ksc = a.k_scale[fp8_scale_index(koff / hd)];
    }
    for (int h = 0; h < G && h < 16; ++h) {
      float sc = kNegInf;
      if (valid) {
        float acc = 0.f;
        for (int d = 0; d < hd; ++d) acc += sq[h * hd + d] * kv_value<K>(a.k_cache, koff + d);
        sc = acc * ksc * a.scale_log2;
      }
      float mx = sc;
      for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      const float m_new = fmaxf(mrun[h], mx);
      const float alpha = __builtin_amdgcn_exp2f(mrun[h] - m_new);
      const float pr = valid ? __builtin_amdgcn_exp2f(sc - m_new) : 0.f;
      float ps = pr;
      for (int off = 32; off > 0; off >>= 1) ps += __shfl_xor(ps, off, 64);
      lrun[h] = lrun[h] * alpha + ps;
      mrun[h] = m_new;
      sp[lane] = pr;
      __builtin_amdgcn_wave_barrier();
      const int nt = min(64, w_end - t0);
      o[h][0] *= alpha;
      o[h][1] *= alpha;
      for (int t = 0; t < nt; ++t) {
        const int64_t voff = token_elem(a, bs, hk, t0 + t, hd);
        float pt = sp[t];
        if constexpr (K == CacheKind::kFP8) pt *= a.v_scale[fp8_scale_index(voff / hd)];
        for (int j = 0; j < 2; ++j)
          if (lane + 64 * j < hd) o[h][j] += pt * kv_value<K>(a.v_cache, voff + lane + 64 * j);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  if (lane < 16) {
    sm[wave * 16 + lane] = kNegInf;
    sl[wave * 16 + lane] = 0.f;
  }
  __builtin_amdgcn_wave_barrier();
  for (int h = 0; h < G && h < 16; ++h) {
    if (lane == 0) {
      sm[wave * 16 + h] = mrun[h];
      sl[wave * 16 + h] = lrun[h];
    }
    for (int j = 0; j < 2; ++j)
      if (lane + 64 * j < hd) so[(wave * G + h) * ws_d + lane + 64 * j] = o[h][j];
  }
  __syncthreads();
  const int64_t item = ((int64_t)b * a.hkv + hk) * a.max_splits + split;
  for (int idx = threadIdx.x; idx < G * hd; idx += kBlockThreads) {
    const int head = idx / hd;
    const int d = idx - head * hd;
    float M = kNegInf;
    for (int w = 0; w < kWavesPerBlock; ++w) M = fmaxf(M, sm[w * 16 + head]);
    float acc = 0.f, lsum = 0.f;
    for (int w = 0; w < kWavesPerBlock; ++w) {
      const float e = __builtin_amdgcn_exp2f(sm[w * 16 + head] - M);
      acc += e * so[(w * G + head) * ws_d + d];
      lsum += e * sl[w * 16 + head];
    }
    a.ws_o[(item * G + head) * ws_d + d] = acc;
    if (d == 0) {
      a.ws_ml[(item * G + head) * 2 + 0] = M;
      a.ws_ml[(item * G + head) * 2 + 1] = lsum;
    }
  }
}

// Merge the splits of one (b, q head): out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s.
// Partial rows are ws_d floats wide; head_dim entries lane + 64 j are written.
template <bool kBF16Out>
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeArgs a, int ws_d) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const int G = a.group;
  const int hk = hq / G;
  const int head = hq - hk * G;
  const int L = min(a.seq_lens[b], a.max_len);
  const int nsplit = L <= 0 ? 0 : (L + a.split_tokens - 1) / a.split_tokens;
  const int64_t item0 = ((int64_t)b * a.hkv + hk) * a.max_splits;
  float M = kNegInf;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, a.ws_ml[((item0 + s) * G + head) * 2]);
  float acc[2] = {0.f, 0.f};
  float lsum = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const int64_t it = (item0 + s) * G + head;
    const float e = __builtin_amdgcn_exp2f(a.ws_ml[it * 2] - M);
    lsum += e * a.ws_ml[it * 2 + 1];
    for (int j = 0; j < 2; ++j)
      if (lane + 64 * j < a.head_dim) acc[j] += e * a.ws_o[it * ws_d + lane + 64 * j];
  }
  const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
  const int64_t dst = (int64_t)b * a.o_sb + (int64_t)hq * a.o_sh;
  for (int j = 0; j < 2; ++j) {
    if (lane + 64 * j >= a.head_dim) continue;
    const float v = acc[j] * inv;
    if constexpr (kBF16Out) {
      static_cast<uint16_t *>(a.out)[dst + lane + 64 * j] = f32_to_bf16_bits(v);
    } else {
      static_cast<float *>(a.out)[dst + lane + 64 * j] = v;
    }
  }
}

template <int D, bool kFP8, bool kPad>
hipError_t launch_mfma(const DecodeArgs &a, dim3 block, size_t lds_merge, hipStream_t stream) {
  const int cus = device_cu_count();
  const int64_t items = (int64_t)a.batch * a.hkv * a.max_splits;  // upper bound of the dense item count
  const dim3 grid((unsigned)std::min<int64_t>(items, (int64_t)cus * 2));
  const size_t lds = (size_t)kWavesPerBlock * Tile<D, kFP8>::kVBytes + lds_merge +
                     sizeof(int) * (kWavesPerBlock + 2 * (size_t)a.batch + 1);
  switch (a.split_tokens / (kWavesPerBlock * kTileTokens)) {
    case 2:
      hipLaunchKernelGGL((decode_split_kernel<D, kFP8, 2, kPad>), grid, block, lds, stream, a);
      break;
    case 4:
      hipLaunchKernelGGL((decode_split_kernel<D, kFP8, 4, kPad>), grid, block, lds, stream, a);
      break;
    case 8:
      hipLaunchKernelGGL((decode_split_kernel<D, kFP8, 8, kPad>), grid, block, lds, stream, a);
      break;
    default:
      hipLaunchKernelGGL((decode_split_kernel<D, kFP8, 1, kPad>), grid, block, lds, stream, a);
      break;
  }
  return hipGetLastError();
}

template <int D, bool kFP8, bool kPad>
hipError_t launch_stream(const DecodeArgs &a0, const DecodeAppend *ap, hipStream_t stream) {
  DecodeArgs a = a0;
  const int64_t blocks = balanced_stream_waves(D, a.batch, a.hkv, a.max_len) / kWavesPerBlock;
  a.stream_waves = (int)(blocks * kWavesPerBlock);
  a.seg_cost = stream_seg_cost(D);
  const size_t lds_prefix = 16 * ((sizeof(int) * (kWavesPerBlock + (size_t)a.batch + 1) + 15) / 16);
  size_t lds = (size_t)kWavesPerBlock * Tile<D, kFP8>::kVBytes + lds_prefix;
  if (ap != nullptr) {
    lds += (size_t)kWavesPerBlock * 16 * D * sizeof(uint16_t);  // q staging
    DecodeAppendArgs f;
    static_cast<DecodeArgs &>(f) = a;
    f.ap = *ap;
    if (ap->part_splits > 0)
      hipLaunchKernelGGL((decode_stream_append_kernel<D, kFP8, true, kPad>), dim3((unsigned)blocks),
                         dim3(64 * kWavesPerBlock), lds, stream, f);
    else
      hipLaunchKernelGGL((decode_stream_append_kernel<D, kFP8, false, kPad>), dim3((unsigned)blocks),
                         dim3(64 * kWavesPerBlock), lds, stream, f);
  } else {
    hipLaunchKernelGGL((decode_stream_kernel<D, kFP8, kPad>), dim3((unsigned)blocks), dim3(64 * kWavesPerBlock), lds,
                       stream, a);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const dim3 mgrid((unsigned)((int64_t)a.batch * a.hkv));
  if (a.group <= 4)
    hipLaunchKernelGGL((decode_merge_kernel<D, 4>), mgrid, dim3(64), 0, stream, a);
  else if (a.group <= 8)
    hipLaunchKernelGGL((decode_merge_kernel<D, 8>), mgrid, dim3(64), 0, stream, a);
  else
    hipLaunchKernelGGL((decode_merge_kernel<D, 16>), mgrid, dim3(64), 0, stream, a);
  return hipGetLastError();
}

template <int D, bool kFP8, bool kPad>
hipError_t launch_segment(const DecodeArgs &a, const DecodeAppend *ap, hipStream_t stream) {
  static_assert(Tile<D, kFP8>::kVBytes * kWavesPerBlock == segment_stream_lds(D, kFP8, false),
                "segment_stream_lds assumes this");
  const dim3 grid((unsigned)segment_grid(a.batch, a.hkv));
  const size_t lds = segment_lds_bytes(D, kFP8, ap != nullptr, a.group);
  if (ap != nullptr) {
    DecodeAppendArgs f;
    static_cast<DecodeArgs &>(f) = a;
    f.ap = *ap;
    if (ap->part_splits > 0)
      hipLaunchKernelGGL((decode_segment_append_kernel<D, kFP8, true, kPad>), grid, dim3(64 * kWavesPerBlock), lds,
                         stream, f);
    else
      hipLaunchKernelGGL((decode_segment_append_kernel<D, kFP8, false, kPad>), grid, dim3(64 * kWavesPerBlock), lds,
                         stream, f);
  } else {
    hipLaunchKernelGGL((decode_segment_kernel<D, kFP8, kPad>), grid, dim3(64 * kWavesPerBlock), lds, stream, a);
  }
  return hipGetLastError();
}

template <int D, bool kFP8, bool kPad>
hipError_t launch_paired(const DecodeArgs &a, const DecodeAppend *ap, hipStream_t stream) {
  constexpr int NWV = paired_waves(D);
  static_assert(Tile<D, kFP8>::kVBytes * NWV == paired_stream_lds(D, kFP8, false, NWV), "paired_stream_lds assumes this");
  const dim3 grid((unsigned)paired_grid(a.batch, a.hkv));
  const size_t lds = paired_lds_bytes(D, kFP8, ap != nullptr, a.group);
  if (lds == 0) return hipErrorInvalidValue;
  if (ap != nullptr) {
    DecodeAppendArgs f;
    static_cast<DecodeArgs &>(f) = a;
    f.ap = *ap;
    if (ap->part_splits > 0)
      hipLaunchKernelGGL((decode_paired_append_kernel<D, kFP8, true, kPad, NWV>), grid, dim3(64 * NWV), lds, stream, f);
    else
      hipLaunchKernelGGL((decode_paired_append_kernel<D, kFP8, false, kPad, NWV>), grid, dim3(64 * NWV), lds, stream,
                         f);
  } else {
    hipLaunchKernelGGL((decode_paired_kernel<D, kFP8, kPad, NWV>), grid, dim3(64 * NWV), lds, stream, a);
  }
  return hipGetLastError();
}

// The one-launch partitions (split_tokens < 0).
template <int D, bool kFP8, bool kPad>
hipError_t launch_onepass(const DecodeArgs &a, const DecodeAppend *ap, hipStream_t stream) {
  if (a.split_tokens == kSplitPaired) return launch_paired<D, kFP8, kPad>(a, ap, stream);
  return launch_segment<D, kFP8, kPad>(a, ap, stream);
}

// MFMA kernels on D-wide tiles (kPad: rows of a.head_dim < D).
template <int D, bool kPad>
hipError_t launch_d(const DecodeArgs &a, CacheKind kind, hipStream_t stream) {
  const dim3 block(64 * kWavesPerBlock);
  const size_t lds = sizeof(float) * (kWavesPerBlock * a.group * D + 2 * kWavesPerBlock * 16);
  hipError_t err = hipSuccess;
  if (kind == CacheKind::kFP8) {
    if constexpr (D >= 64) {  // fp8 tiles are at least 64 wide (one 16-byte fragment per lane and row)
      if (a.split_tokens < 0) return launch_onepass<D, true, kPad>(a, nullptr, stream);
      if (a.split_tokens == 0) return launch_stream<D, true, kPad>(a, nullptr, stream);
      err = launch_mfma<D, true, kPad>(a, block, lds, stream);
    } else {
      return hipErrorInvalidValue;
    }
  } else {
    if (a.split_tokens < 0) return launch_onepass<D, false, kPad>(a, nullptr, stream);
    if (a.split_tokens == 0) return launch_stream<D, false, kPad>(a, nullptr, stream);
    err = launch_mfma<D, false, kPad>(a, block, lds, stream);
  }
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((decode_combine_kernel<true>), dim3(a.hq, a.batch), dim3(64), 0, stream, a, D);
  return hipGetLastError();
}

hipError_t launch_valu(const DecodeArgs &a, CacheKind kind, hipStream_t stream) {
  const int ws_d = workspace_head_dim(a.head_dim, kind);
  const dim3 grid(a.max_splits, a.hkv, a.batch);
  const dim3 block(64 * kWavesPerBlock);
  const size_t lds = sizeof(float) * (kWavesPerBlock * a.group * ws_d + 2 * kWavesPerBlock * 16 +
                                      a.group * a.head_dim + kWavesPerBlock * 64);
  switch (kind) {
    case CacheKind::kF32:
      hipLaunchKernelGGL((decode_split_kernel_valu<CacheKind::kF32>), grid, block, lds, stream, a, ws_d);
      break;
    case CacheKind::kBF16:
      hipLaunchKernelGGL((decode_split_kernel_valu<CacheKind::kBF16>), grid, block, lds, stream, a, ws_d);
      break;
    case CacheKind::kFP8:
      hipLaunchKernelGGL((decode_split_kernel_valu<CacheKind::kFP8>), grid, block, lds, stream, a, ws_d);
      break;
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  if (kind == CacheKind::kF32)
    hipLaunchKernelGGL((decode_combine_kernel<false>), dim3(a.hq, a.batch), dim3(64), 0, stream, a, ws_d);
  else
    hipLaunchKernelGGL((decode_combine_kernel<true>), dim3(a.hq, a.batch), dim3(64), 0, stream, a, ws_d);
  return hipGetLastError();
}

}  // namespace

int64_t balanced_stream_waves(int head_dim, int64_t batch, int64_t hkv, int64_t max_len) {
  // stream_blocks_per_cu(D) resident workgroups of 4 waves per CU; no more waves than the longest-case tile count
  const int64_t tiles_bound = batch * hkv * ((max_len + kTileTokens - 1) / kTileTokens);
  int64_t blocks = std::min<int64_t>((int64_t)device_cu_count() * stream_blocks_per_cu(head_dim), kMaxStreamBlocks);
  blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, (tiles_bound + kWavesPerBlock - 1) / kWavesPerBlock));
  return blocks * kWavesPerBlock;
}

int64_t segment_grid(int64_t batch, int64_t hkv) { return batch * hkv; }

size_t segment_lds_bytes(int tile_d, bool fp8, bool fused, int64_t group) {
  const int g = (int)group;
  const int stream = segment_stream_lds(tile_d, fp8, fused), merge = segment_merge_lds(tile_d, g);
  return (size_t)(segment_merge_separate(tile_d, fp8, fused, g) ? stream + merge : (stream > merge ? stream : merge));
}

int64_t paired_grid(int64_t batch, int64_t hkv) { return (batch + 1) / 2 * hkv; }

size_t paired_lds_bytes(int tile_d, bool fp8, bool fused, int64_t group) {
  if (group < 1 || group > 16) return 0;
  const int bytes = paired_lds(tile_d, fp8, fused, (int)group, paired_waves(tile_d));
  return bytes <= 65536 ? (size_t)bytes : 0;
}

int64_t segment_round(int tile_d) { return (int64_t)device_cu_count() * stream_blocks_per_cu(tile_d); }

int64_t auto_split_tokens(int64_t batch, int64_t hkv, int64_t max_len) {
  // Aim for >= 8 workgroups per CU (256 CUs) over the longest sequence while
  // keeping splits long enough that the partial write (G*(D+2) floats) stays
  // a small fraction of the K/V bytes a split reads.
  const int64_t target_blocks = 256 * 8;
  int64_t split = 1024;
  while (split > 128 && batch * hkv * ((max_len + split - 1) / split) < target_blocks) split /= 2;
  return split;
}

hipError_t launch_decode_attn(const DecodeArgs &a, CacheKind kind, int head_dim, hipStream_t stream) {
  const int D = tile_head_dim(head_dim, kind);
  const bool pad = D != head_dim;
  // row attention (a row -> sequence map) exists only in the VALU kernel; the
  // MFMA kernels address the cache by row index and must never see it
  if (D == 0 || a.seq_of_row != nullptr) return launch_valu(a, kind, stream);
  if (D == 32) return pad ? launch_d<32, true>(a, kind, stream) : launch_d<32, false>(a, kind, stream);
  if (D == 64) return pad ? launch_d<64, true>(a, kind, stream) : launch_d<64, false>(a, kind, stream);
  return pad ? launch_d<128, true>(a, kind, stream) : launch_d<128, false>(a, kind, stream);
}

hipError_t launch_decode_attn_append(const DecodeAppendArgs &a, CacheKind kind, int head_dim, hipStream_t stream) {
  const int D = tile_head_dim(head_dim, kind);
  const bool pad = D != head_dim;
  if (a.split_tokens < 0) {
    if (kind == CacheKind::kFP8) {
      if (D == 64) return pad ? launch_onepass<64, true, true>(a, &a.ap, stream) : launch_onepass<64, true, false>(a, &a.ap, stream);
      if (D == 128) return pad ? launch_onepass<128, true, true>(a, &a.ap, stream) : launch_onepass<128, true, false>(a, &a.ap, stream);
      return hipErrorInvalidValue;
    }
    if (D == 32) return pad ? launch_onepass<32, false, true>(a, &a.ap, stream) : launch_onepass<32, false, false>(a, &a.ap, stream);
    if (D == 64) return pad ? launch_onepass<64, false, true>(a, &a.ap, stream) : launch_onepass<64, false, false>(a, &a.ap, stream);
    if (D == 128) return pad ? launch_onepass<128, false, true>(a, &a.ap, stream) : launch_onepass<128, false, false>(a, &a.ap, stream);
    return hipErrorInvalidValue;
  }
  if (kind == CacheKind::kFP8) {
    if (D == 64) return pad ? launch_stream<64, true, true>(a, &a.ap, stream) : launch_stream<64, true, false>(a, &a.ap, stream);
    if (D == 128) return pad ? launch_stream<128, true, true>(a, &a.ap, stream) : launch_stream<128, true, false>(a, &a.ap, stream);
    return hipErrorInvalidValue;
  }
  if (D == 32) return pad ? launch_stream<32, false, true>(a, &a.ap, stream) : launch_stream<32, false, false>(a, &a.ap, stream);
  if (D == 64) return pad ? launch_stream<64, false, true>(a, &a.ap, stream) : launch_stream<64, false, false>(a, &a.ap, stream);
  if (D == 128) return pad ? launch_stream<128, false, true>(a, &a.ap, stream) : launch_stream<128, false, false>(a, &a.ap, stream);
  return hipErrorInvalidValue;
}

}  // namespace tt
