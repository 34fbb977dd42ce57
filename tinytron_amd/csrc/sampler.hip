// Token sampling on gfx950: tinytron/inference/sampler.py:6-62 in one launch.
//
// One 1024-thread workgroup per row of logits [M, V] (V <= 65536 bf16,
// 32768 fp32). The row lives in registers (thread t holds the 8-element
// groups 8 (t + 1024 g) .. + 7, so a group load is one 16- or 32-byte access
// and the index order is (g, thread, element)). Steps, all inside the
// workgroup:
//
//   y = float(x) / temperature          (sampler.py:16-18; skipped at 1.0)
//   max, first argmax, tie count        (one block reduction)
//   top-k  (sampler.py:20-24): keep y >= the k-th largest value, counting
//          duplicates. The k-th largest is found by an MSB-first radix
//          select over order-preserving 32-bit keys of y (four 8-bit digit
//          passes, integer histograms in LDS).
//   top-p  (sampler.py:26-34): sorted descending, a token is kept when the
//          cumulative probability up to and including it is <= p, the first
//          always kept. The masses exp(y - max) are held as 2^-40 fixed
//          point (exact 64-bit integer sums, so the result does not depend
//          on summation order); a radix select over the keys weighted by
//          mass finds the boundary value kb = the largest value whose
//          cumulative mass exceeds p. Values above kb are kept; of the
//          tokens equal to kb the first r in index order are kept (the
//          order a stable descending sort gives), r from the mass above kb.
//   log_softmax of the filtered logits (sampler.py:56): (y - max) - log(Z),
//          Z = sum over kept tokens of exp(y - max) in a fixed order.
//   draw   top_k == 1: the first maximum (the reference draws among exactly
//          tied maxima at random). Otherwise inverse CDF in index order over
//          the kept fixed-point masses with a 64-bit uniform from SplitMix64
//          (Steele, Lea and Flood, 2014) keyed by (seed, offset, row): the same
//          distribution as torch.multinomial over softmax(filtered), not the
//          same random stream.
//
// Candidate path (2 <= top_k <= kCandSlots, no full log-probability rows,
// V > kCandChunk): one workgroup per row leaves most CUs idle, so the row is
// first cut into kCandChunk-logit chunks, each reduced on a workgroup of its
// own to its top-k candidates (topk_candidates_kernel: the values >= the
// chunk's k-th largest). The row's kept set lies within the union of those
// (the row's k-th largest is >= every chunk's), so one wave then finishes the
// row on at most kCandSlots x chunks candidates (candidates_pick) with the
// same rules and the same fixed-point masses as the whole-row path. A row the
// candidates cannot decide exactly -- ties at the row's boundary that a chunk
// had no slots for, more than kCandSlots kept tokens, fewer than k finite
// logits -- runs the whole-row path in the same launch.
#include <climits>

#include "tt_internal.h"

namespace tt {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr float kMassScale = 1099511627776.0f;  // 2^40
typedef unsigned long long u64;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Radix histograms are replicated kRep times, replica = lane mod kRep: the
// top digit of the keys of a logit row falls in a handful of bins, and a
// wave's 64 same-address LDS atomics would serialise; with the replicas at
// adjacent addresses a wave instruction makes at most 64 / kRep same-address
// updates. The replicas are summed into hist before a digit is picked.
constexpr int kRep = 16;

struct SampleShared {
  u64 hist[256];
  u64 hrep[256 * kRep];  // [bin][replica]
  u64 red[kWaves][8];
  float fv[kWaves];
  int iv[kWaves];
  int cv[kWaves];
  int nv[kWaves];
  u64 bc[4];
};

// Order-preserving key: key(a) < key(b) iff a < b for non-NaN floats
// (-0 is folded into +0, which compares equal to it).
__device__ __forceinline__ uint32_t order_key(float y) {
  const uint32_t b = __float_as_uint(y == 0.f ? 0.f : y);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ u64 splitmix64_mix(u64 z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// 64-bit uniform of (seed, offset, row): three chained SplitMix64 outputs.
__device__ __forceinline__ u64 draw_u64(u64 seed, u64 offset, u64 row) {
  constexpr u64 kGamma = 0x9E3779B97F4A7C15ull;
  u64 h = splitmix64_mix(seed + kGamma);
  h = splitmix64_mix(h + (offset + 1) * kGamma);
  return splitmix64_mix(h + (row + 1) * kGamma);
}

__device__ __forceinline__ u64 mass_of(float y, float m) {
  return (u64)rintf(expf(y - m) * kMassScale);
}

__device__ __forceinline__ u64 wave_sum_u64(u64 v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ u64 block_sum_u64(u64 v, SampleShared &sh) {
  v = wave_sum_u64(v);
  if ((threadIdx.x & 63) == 0) sh.red[threadIdx.x >> 6][0] = v;
  __syncthreads();
  u64 t = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t += sh.red[w][0];
  __syncthreads();
  return t;
}

// Sum in a fixed order: thread-sequential, xor butterfly, waves ascending.
__device__ __forceinline__ float block_sum_f32(float v, SampleShared &sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) sh.fv[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t += sh.fv[w];
  __syncthreads();
  return t;
}

// Wave 0: the largest digit d with sum_{d' >= d} hist[d'] >= need (the caller
// guarantees the total reaches need); bc[0] = d, bc[1] = sum over d' > d.
__device__ __forceinline__ void pick_digit(SampleShared &sh, u64 need) {
  const int lane = threadIdx.x & 63;
  u64 h[4];
  u64 s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = sh.hist[255 - 4 * lane - j];
    s += h[j];
  }
  u64 incl = s;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const u64 o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  const u64 excl = incl - s;
  if (incl >= need && excl < need) {
    u64 c = excl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (c + h[j] >= need) {
        sh.bc[0] = (u64)(255 - 4 * lane - j);
        sh.bc[1] = c;
        break;
      }
      c += h[j];
    }
  }
}

// The row as this thread holds it: fp32 values, or (bf16 logits) the raw
// bf16 pairs, two per register, converted and divided by the temperature at
// each use (the division is exact-rounded, so every pass sees the same y).
template <int EPT, bool kF32>
struct Row {
  static constexpr int kRegs = kF32 ? EPT : EPT / 2;
  uint32_t w[kRegs];
  int t;  // thread index
  int V;
  int apply_temp;
  float temperature;
  __device__ __forceinline__ int index(int g, int e) const { return 8 * (t + kThreads * g) + e; }
  __device__ __forceinline__ float val(int j) const {
    float x;
    if (kF32)
      x = __uint_as_float(w[j]);
    else
      x = __uint_as_float((j & 1) ? (w[j >> 1] & 0xffff0000u) : (w[j >> 1] << 16));
    return apply_temp ? x / temperature : x;
  }
  // Start of a pass over the row: the values and the thread index count as
  // redefined here, so the compiler recomputes keys, masses and index
  // comparisons per pass instead of keeping them all live across passes
  // (which would not fit in the register budget).
  __device__ __forceinline__ void pass() {
#pragma unroll
    for (int j = 0; j < kRegs; ++j) asm volatile("" : "+v"(w[j]));
    asm volatile("" : "+v"(t));
  }
};

// MSB-first radix select over the keys weighted by wfn(idx, y) (zero for
// the -inf padding past V): the largest key kb with sum_{key >= kb} weight
// >= need.
// above = sum_{key > kb} weight, at = sum_{key == kb} weight.
template <int EPT, bool kF32, class WeightFn>
__device__ __forceinline__ uint32_t radix_select(SampleShared &sh, Row<EPT, kF32> &r, u64 need, WeightFn wfn,
                                                 u64 &above, u64 &at) {
  uint32_t prefix = 0, mask = 0;
  above = 0;
  at = 0;
  const uint32_t rep = threadIdx.x & (kRep - 1);
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256 * kRep; i += kThreads) sh.hrep[i] = 0;
    __syncthreads();
    r.pass();
#pragma unroll
    for (int g = 0; g < EPT / 8; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int idx = r.index(g, e);
        const float v = r.val(8 * g + e);
        const uint32_t key = order_key(v);
        if ((key & mask) == prefix) {
          const u64 w = wfn(idx, v);
          if (w) atomicAdd(&sh.hrep[((key >> shift) & 255u) * kRep + rep], w);
        }
      }
    __syncthreads();
    if (threadIdx.x < 256) {  // replica sums; the rotated start spreads the reads over the banks
      u64 t = 0;
#pragma unroll
      for (int j = 0; j < kRep; ++j) t += sh.hrep[threadIdx.x * kRep + ((j + threadIdx.x) & (kRep - 1))];
      sh.hist[threadIdx.x] = t;
    }
    __syncthreads();
    if (threadIdx.x < 64) pick_digit(sh, need);
    __syncthreads();
    const uint32_t d = (uint32_t)sh.bc[0];
    const u64 ab = sh.bc[1];
    at = sh.hist[d];
    above += ab;
    need -= ab;
    prefix |= d << shift;
    mask |= 0xFFu << shift;
    __syncthreads();
  }
  return prefix;
}

// First index (in index order) at which the running sum of wfn(idx, y)
// exceeds target (weights zero for the -inf padding); the caller guarantees
// target < the total.
template <int EPT, bool kF32, class WeightFn>
__device__ __forceinline__ int find_first_exceeding(SampleShared &sh, Row<EPT, kF32> &r, u64 target, WeightFn wfn) {
  constexpr int G = EPT / 8;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  u64 s[G];
  r.pass();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    s[g] = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[g] += wfn(r.index(g, e), r.val(8 * g + e));
    }
    const u64 t = wave_sum_u64(s[g]);
    if (lane == 0) sh.red[wave][g] = t;
  }
  __syncthreads();
  int gs = -1, ws = -1;
  u64 cum = 0;
#pragma unroll 1
  for (int g = 0; g < G && gs < 0; ++g)
#pragma unroll 1
    for (int w = 0; w < kWaves; ++w) {
      const u64 t = sh.red[w][g];
      if (cum + t > target) {
        gs = g;
        ws = w;
        break;
      }
      cum += t;
    }
  if (wave == ws) {
    const u64 rel = target - cum;
    u64 sv = 0;
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (g == gs) sv = s[g];
    u64 incl = sv;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const u64 o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    const u64 excl = incl - sv;
    if (incl > rel && excl <= rel) {
      r.pass();
      u64 c = excl;
      int found = -1;
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (g == gs) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int idx = r.index(g, e);
            const u64 w = wfn(idx, r.val(8 * g + e));
            if (found < 0 && c + w > rel) found = idx;
            c += w;
          }
        }
      sh.bc[2] = (u64)found;
    }
  }
  __syncthreads();
  const int res = (int)sh.bc[2];
  __syncthreads();
  return res;
}

// The row into registers; elements past V read nothing and hold -inf. Every
// full group's vector load is issued before any is used (a partial or empty
// group loads the row's first group instead, always in bounds), so the row
// costs one memory round trip; the one partial group of the row then reads
// its elements one by one.
template <int EPT, bool kF32>
__device__ __forceinline__ void load_row(const SampleArgs &a, int row, Row<EPT, kF32> &r) {
  constexpr int G = EPT / 8;
  r.t = threadIdx.x;
  r.V = a.V;
  r.apply_temp = a.apply_temp;
  r.temperature = a.temperature;
  const char *rowp = static_cast<const char *>(a.logits) + (int64_t)row * a.ld * (kF32 ? 4 : 2);
  if (a.vec) {
    constexpr int kVec = kF32 ? 2 : 1;  // 16-byte loads per group
    u32x4 raw[G][kVec];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int base = r.index(g, 0);
      const char *src = rowp + (base + 8 <= a.V ? base : 0) * (kF32 ? 4 : 2);
#pragma unroll
      for (int h = 0; h < kVec; ++h) raw[g][h] = *reinterpret_cast<const u32x4 *>(src + 16 * h);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int base = r.index(g, 0);
      if (base + 8 <= a.V) {
#pragma unroll
        for (int h = 0; h < kVec; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e) r.w[(kF32 ? 8 : 4) * g + 4 * h + e] = raw[g][h][e];
      } else {
#pragma unroll
        for (int j = 0; j < Row<EPT, kF32>::kRegs / G; ++j) r.w[(Row<EPT, kF32>::kRegs / G) * g + j] = kF32 ? 0xff800000u : 0xff80ff80u;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < Row<EPT, kF32>::kRegs; ++j) r.w[j] = kF32 ? 0xff800000u : 0xff80ff80u;
  }
  // The partial group (at most one per row), or every group for rows that
  // are not 16-byte aligned: element loads.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int base = r.index(g, 0);
    if ((!a.vec && base < a.V) || (base < a.V && base + 8 > a.V)) {
      if (kF32) {
        const float *src = reinterpret_cast<const float *>(rowp) + base;
#pragma unroll
        for (int e = 0; e < 8; ++e) r.w[8 * g + e] = base + e < a.V ? __float_as_uint(src[e]) : 0xff800000u;
      } else {
        const uint16_t *src = reinterpret_cast<const uint16_t *>(rowp) + base;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = base + 2 * e < a.V ? src[2 * e] : 0xff80u;
          const uint32_t hi = base + 2 * e + 1 < a.V ? src[2 * e + 1] : 0xff80u;
          r.w[4 * g + e] = lo | (hi << 16);
        }
      }
    }
  }
}

struct RowMax {
  float m;      // maximum
  int amax;     // its first index
  int cmax;     // its multiplicity
  int nfinite;  // finite values in the row
};

// Block reduction of the row's maximum, first argmax and tie count.
template <int EPT, bool kF32>
__device__ __forceinline__ RowMax row_max(const SampleArgs &a, const Row<EPT, kF32> &r, SampleShared &sh) {
  constexpr int G = EPT / 8;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float bm = -INFINITY;
  int bi = INT_MAX, bcnt = 0, nfin = 0;
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int idx = r.index(g, e);
      const float v = r.val(8 * g + e);
      if (idx < a.V) {
        nfin += v > -INFINITY;
        if (bi == INT_MAX || v > bm) {
          bm = v;
          bi = idx;
          bcnt = 1;
        } else if (v == bm) {
          ++bcnt;
        }
      }
    }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bm, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    const int oc = __shfl_xor(bcnt, off, 64);
    nfin += __shfl_xor(nfin, off, 64);
    if (ov > bm || (bi == INT_MAX && oi != INT_MAX)) {
      bm = ov;
      bi = oi;
      bcnt = oc;
    } else if (ov == bm && oi != INT_MAX) {
      bi = oi < bi ? oi : bi;
      bcnt += oc;
    }
  }
  if (lane == 0) {
    sh.fv[wave] = bm;
    sh.iv[wave] = bi;
    sh.cv[wave] = bcnt;
    sh.nv[wave] = nfin;
  }
  __syncthreads();
  float m = -INFINITY;
  int amax = INT_MAX, cmax = 0, nfinite = 0;
#pragma unroll 1
  for (int w = 0; w < kWaves; ++w) {
    nfinite += sh.nv[w];
    const float ov = sh.fv[w];
    const int oi = sh.iv[w];
    if (oi == INT_MAX) continue;
    if (amax == INT_MAX || ov > m) {
      m = ov;
      amax = oi;
      cmax = sh.cv[w];
    } else if (ov == m) {
      amax = oi < amax ? oi : amax;
      cmax += sh.cv[w];
    }
  }
  __syncthreads();
  return RowMax{m, amax, cmax, nfinite};
}

// ---- candidate path ----------------------------------------------------------

constexpr int kCandThreads = 256;
constexpr int kCandEPT = kCandChunk / kCandThreads;  // 32 logits per thread, 8-logit groups

struct CandShared {
  uint32_t hrep[2][256 * kRep];  // [pass parity][bin][replica]
  uint32_t hist[256];
  uint32_t bc[3];
  int cnt;
};

// Workgroup (chunk c, row): the chunk's logits in registers (thread t holds
// groups 8 (t + 256 g) .. + 7 of the chunk), the k-th largest order key by
// MSB-first radix select (integer histograms in LDS, replicated as in
// radix_select), then the candidates: every value strictly above it (fewer
// than k of them), then values equal to it while slots remain.
template <bool kF32>
__global__ __launch_bounds__(kCandThreads) void topk_candidates_kernel(SampleArgs a) {
  __shared__ CandShared sh;
  constexpr int G = kCandEPT / 8;
  const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
  const int base = c * kCandChunk;
  CandRecord *rec = static_cast<CandRecord *>(a.cand) + (int64_t)row * a.cand_chunks + c;
  const char *rowp = static_cast<const char *>(a.logits) + (int64_t)row * a.ld * (kF32 ? 4 : 2);

  // loads: every full group's vector load issued before any is used; the
  // partial group (at most one per row) or unaligned rows read element by element
  constexpr int kVec = kF32 ? 2 : 1;
  u32x4 raw[G][kVec];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int i0 = base + 8 * (t + kCandThreads * g);
    const bool full = a.vec && i0 + 8 <= a.V;
    const char *src = rowp + (int64_t)(full ? i0 : 0) * (kF32 ? 4 : 2);
#pragma unroll
    for (int h = 0; h < kVec; ++h) raw[g][h] = full ? *reinterpret_cast<const u32x4 *>(src + 16 * h) : u32x4{0, 0, 0, 0};
  }
  float y[kCandEPT];
  uint32_t key[kCandEPT];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int i0 = base + 8 * (t + kCandThreads * g);
    const bool full = a.vec && i0 + 8 <= a.V;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x;
      if (full) {
        const uint32_t w = raw[g][kF32 ? e / 4 : 0][kF32 ? e % 4 : e / 2];
        x = kF32 ? __uint_as_float(w) : __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
      } else if (i0 + e < a.V) {
        x = kF32 ? reinterpret_cast<const float *>(rowp)[i0 + e]
                 : __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(rowp)[i0 + e] << 16);
      } else {
        x = -INFINITY;
      }
      y[8 * g + e] = a.apply_temp ? x / a.temperature : x;
      key[8 * g + e] = i0 + e < a.V ? order_key(y[8 * g + e]) : 0u;  // real keys are >= key(-inf) > 0
    }
  }

  const int nvalid = a.V - base < kCandChunk ? a.V - base : kCandChunk;
  // kth: the chunk's k-th largest key, or (early) a lower bound of it below
  // which at most kCandSlots keys lie at or above; the candidates are then all
  // keys >= it. The select stops after a digit once the keys at or above its
  // bin fit in the slots (with logit rows this is usually after 16 bits).
  uint32_t kth = 1;  // below every real key: all of a chunk with at most k logits are candidates
  bool all_fit = true;
  if (nvalid > a.top_k) {
    uint32_t prefix = 0, mask = 0, need = (uint32_t)a.top_k, above = 0;
    const uint32_t rep = t & (kRep - 1);
    for (int i = t; i < 256 * kRep; i += kCandThreads) sh.hrep[0][i] = 0;
    __syncthreads();
#pragma unroll 1
    for (int shift = 24, pass = 0; shift >= 0; shift -= 8, ++pass) {
      uint32_t *hr = sh.hrep[pass & 1];
#pragma unroll
      for (int j = 0; j < kCandEPT; ++j)
        if (key[j] != 0u && (key[j] & mask) == prefix) atomicAdd(&hr[((key[j] >> shift) & 255u) * kRep + rep], 1u);
      __syncthreads();
      {
        uint32_t h = 0;
#pragma unroll
        for (int j = 0; j < kRep; ++j) h += hr[t * kRep + ((j + t) & (kRep - 1))];
        sh.hist[t] = h;
        uint32_t *nx = sh.hrep[(pass + 1) & 1];  // the next pass's histogram, unused since the last barrier
        for (int i = t; i < 256 * kRep; i += kCandThreads) nx[i] = 0;
      }
      __syncthreads();
      if (t < 64) {  // the largest digit whose suffix count reaches need
        uint32_t h[4], sum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h[j] = sh.hist[255 - 4 * t - j];
          sum += h[j];
        }
        uint32_t incl = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const uint32_t o = __shfl_up(incl, off, 64);
          if (t >= off) incl += o;
        }
        const uint32_t excl = incl - sum;
        if (incl >= need && excl < need) {
          uint32_t cum = excl;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (cum + h[j] >= need) {
              sh.bc[0] = 255u - 4u * t - j;
              sh.bc[1] = cum;
              sh.bc[2] = h[j];
              break;
            }
            cum += h[j];
          }
        }
      }
      __syncthreads();
      need -= sh.bc[1];
      above += sh.bc[1];
      prefix |= sh.bc[0] << shift;
      mask |= 0xFFu << shift;
      if (above + sh.bc[2] <= (uint32_t)kCandSlots) break;  // every key >= prefix fits: uniform exit
      if (shift == 0) all_fit = false;
    }
    kth = prefix;
  }

  if (t == 0) sh.cnt = 0;
  __syncthreads();
  if (all_fit) {  // every real key >= kth, at most kCandSlots of them
#pragma unroll
    for (int j = 0; j < kCandEPT; ++j)
      if (key[j] != 0u && key[j] >= kth) {
        const int slot = atomicAdd(&sh.cnt, 1);
        rec->val[slot] = y[j];
        rec->idx[slot] = base + 8 * (t + kCandThreads * (j / 8)) + j % 8;
      }
  } else {  // kth is the k-th largest key: the keys above it (fewer than k), then its ties while slots remain
#pragma unroll
    for (int j = 0; j < kCandEPT; ++j)
      if (key[j] > kth) {
        const int slot = atomicAdd(&sh.cnt, 1);
        rec->val[slot] = y[j];
        rec->idx[slot] = base + 8 * (t + kCandThreads * (j / 8)) + j % 8;
      }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kCandEPT; ++j)
      if (key[j] == kth) {
        const int slot = atomicAdd(&sh.cnt, 1);
        if (slot < kCandSlots) {
          rec->val[slot] = y[j];
          rec->idx[slot] = base + 8 * (t + kCandThreads * (j / 8)) + j % 8;
        }
      }
  }
  __syncthreads();
  if (t == 0) {
    rec->count = sh.cnt < kCandSlots ? sh.cnt : kCandSlots;
    rec->truncated = sh.cnt > kCandSlots;
    rec->kth_key = kth;
  }
}

// Wave 0 of a row's sample_kernel workgroup: the row's result from its
// chunks' candidates when they decide it exactly (returns false otherwise,
// writing nothing). Lane l reads slot l of every chunk. Counting and ranking
// go through ballots and lane reads (scalar), not LDS shuffles: every step
// here is a short dependent chain.
__device__ __forceinline__ u64 lane_u64(u64 v, int j) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, j);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), j);
  return ((u64)hi << 32) | lo;
}

__device__ __forceinline__ bool candidates_pick(const CandRecord *rec, int P, int k, int apply_top_p, float top_p,
                                                u64 seed, u64 offset, int row, int64_t *tokens, float *token_logprob,
                                                SampleShared &sh) {
  const int lane = threadIdx.x;  // P <= kMaxSampleVocabBF16 / kCandChunk = 8 chunks
  rec += (int64_t)row * P;
  constexpr int kMaxChunks = kMaxSampleVocabBF16 / kCandChunk;
  // every record's header and slot are loaded at once (chunks past P re-read
  // chunk 0; slots past a count hold stale data and are masked below): one
  // memory round trip
  int cnt[kMaxChunks], trunc[kMaxChunks];
  uint32_t kthk[kMaxChunks], key[kMaxChunks];
  float val[kMaxChunks];
  int idx[kMaxChunks];
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const CandRecord &rc = rec[c < P ? c : 0];
    cnt[c] = rc.count;
    trunc[c] = rc.truncated;
    kthk[c] = rc.kth_key;
    val[c] = rc.val[lane];
    idx[c] = rc.idx[lane];
  }
  int nvalid = 0;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const bool valid = c < P && lane < cnt[c];
    key[c] = valid ? order_key(val[c]) : 0u;
    if (!valid) {
      val[c] = -INFINITY;
      idx[c] = INT_MAX;
    }
    nvalid += __popcll(__ballot(valid));
  }
  if (nvalid < k) return false;
  // the row's k-th largest key: the largest thr with #(key >= thr) >= k
  uint32_t thr = 0;
#pragma unroll 1
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t trial = thr | (1u << bit);
    int n = 0;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) n += __popcll(__ballot(key[c] >= trial));
    if (n >= k) thr = trial;
  }
  if (thr <= order_key(-INFINITY)) return false;  // fewer than k finite logits
  bool tied_out = false;  // kept ties beyond a chunk's slots
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) tied_out |= c < P && trunc[c] && kthk[c] == thr;
  if (tied_out) return false;
  u64 kmask[kMaxChunks];
  int total = 0;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    kmask[c] = __ballot(key[c] >= thr);
    total += __popcll(kmask[c]);
  }
  if (total > 64) return false;

  // compact the kept candidates to one per lane: (key desc, index asc) as one
  // 64-bit sort key, and the value
  u64 *ck = sh.hrep;
  u64 *cv = sh.hrep + 64;
  const u64 below_lane = (1ull << lane) - 1ull;
  int base = 0;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    if (key[c] >= thr) {
      const int pos = base + __popcll(kmask[c] & below_lane);
      ck[pos] = ((u64)key[c] << 32) | (u64)(0xFFFFFFFFu - (uint32_t)idx[c]);
      cv[pos] = (u64)__float_as_uint(val[c]);
    }
    base += __popcll(kmask[c]);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const bool in = lane < total;
  const u64 sk = in ? ck[lane] : 0ull;
  const float v = in ? __uint_as_float((uint32_t)cv[lane]) : -INFINITY;
  const int my_idx = in ? (int)(0xFFFFFFFFu - (uint32_t)sk) : INT_MAX;
  // rank in (value desc, index asc) order
  int rank = 0;
#pragma unroll 1
  for (int j = 0; j < total; ++j) rank += lane_u64(sk, j) > sk;
  const int top = __builtin_ctzll(__ballot(in && rank == 0));
  const float m = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, v), top));
  const u64 mass = in ? mass_of(v, m) : 0ull;
  bool keep = in;
  if (apply_top_p) {  // in rank order: keep while the cumulative mass stays <= T; the first always
    u64 etot = 0, cum = 0;
#pragma unroll 1
    for (int j = 0; j < total; ++j) {
      const u64 mj = lane_u64(mass, j);
      etot += mj;
      if (__builtin_amdgcn_readlane(rank, j) <= rank) cum += mj;
    }
    const u64 T = (u64)((double)top_p * (double)etot);
    keep = in && (cum <= T || rank == 0);
  }
  // log Z in rank order (a fixed order: the slots' order within a chunk is not)
  const float e = keep ? expf(v - m) : 0.f;
  float z = 0.f;
#pragma unroll 1
  for (int r = 0; r < total; ++r) {
    const int l = __builtin_ctzll(__ballot(in && rank == r));
    z += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, e), l));
  }
  const float logz = logf(z);
  // inverse CDF in index order over the kept masses
  const u64 w = keep ? mass : 0ull;
  u64 wtot = 0, below = 0;  // below: kept mass at indices <= this lane's
#pragma unroll 1
  for (int j = 0; j < total; ++j) {
    const u64 wj = lane_u64(w, j);
    wtot += wj;
    if (__builtin_amdgcn_readlane(my_idx, j) <= my_idx) below += wj;
  }
  const u64 target = __umul64hi(draw_u64(seed, offset, (u64)row), wtot);
  int cand = keep && w > 0 && below > target ? my_idx : INT_MAX;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int o = __shfl_xor(cand, off, 64);
    cand = o < cand ? o : cand;
  }
  if (my_idx == cand && keep) {
    tokens[row] = cand;
    if (token_logprob) token_logprob[row] = (v - m) - logz;
  }
  return true;
}

template <int EPT, bool kF32>
__global__ __launch_bounds__(kThreads) void sample_kernel(SampleArgs a) {
  __shared__ SampleShared sh;
  constexpr int G = EPT / 8;
  const int row = blockIdx.x;
  if (a.cand != nullptr) {
    if (threadIdx.x < 64) {
      const bool done = candidates_pick(static_cast<const CandRecord *>(a.cand), a.cand_chunks, a.top_k,
                                        a.apply_top_p, a.top_p, a.seed, a.offset, row, a.tokens, a.token_logprob, sh);
      if (threadIdx.x == 0) sh.iv[0] = done;
    }
    __syncthreads();
    const bool done = sh.iv[0] != 0;
    __syncthreads();
    if (done) return;
  }
  Row<EPT, kF32> r;
  load_row<EPT, kF32>(a, row, r);
  const RowMax mx = row_max<EPT, kF32>(a, r, sh);
  const float m = mx.m;
  const int amax = mx.amax, cmax = mx.cmax, nfinite = mx.nfinite;

  const bool greedy = a.top_k == 1;
  const bool do_topk = a.top_k > 0 && a.top_k < a.V;
  const bool fast = greedy && cmax == 1;

  // top-k threshold key (0 keeps every element). With at most k finite
  // values the k-th largest is the smallest finite one or -inf, and every
  // finite value is kept.
  uint32_t thrk = 0;
  if (do_topk && !fast) {
    if (greedy) {
      thrk = order_key(m);
    } else if (nfinite > a.top_k) {
      u64 ab, at;
      thrk = radix_select(
          sh, r, (u64)a.top_k, [](int, float v) { return v > -INFINITY ? (u64)1 : (u64)0; }, ab, at);
    }
  }
  auto kept_k = [&](float v) { return order_key(v) >= thrk; };

  // top-p boundary: keys above kb kept, key == kb kept up to index ir.
  uint32_t kb = 0;
  int ir = INT_MAX;
  const bool do_topp = a.apply_top_p && !fast;
  if (do_topp) {
    u64 local = 0;
    r.pass();
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = r.val(8 * g + e);
        if (kept_k(v)) local += mass_of(v, m);
      }
    const u64 etot = block_sum_u64(local, sh);
    const u64 T = (u64)((double)a.top_p * (double)etot);
    u64 ab, at;
    kb = radix_select(
        sh, r, T + 1, [&](int, float v) { return kept_k(v) ? mass_of(v, m) : (u64)0; }, ab, at);
    const u64 eb = mass_of(key_value(kb), m);
    u64 keep_n = eb > 0 && T >= ab ? (T - ab) / eb : 0;
    if (ab == 0 && keep_n == 0) keep_n = 1;  // the first sorted token is always kept
    if (keep_n == 0) {
      ir = -1;
    } else if (eb > 0 && keep_n < at / eb) {
      ir = find_first_exceeding(sh, r, keep_n - 1, [&](int, float v) {
        return (kept_k(v) && order_key(v) == kb) ? (u64)1 : (u64)0;
      });
    }
  }
  auto keep = [&](int idx, float v) {
    if (fast) return idx == amax;
    if (!kept_k(v)) return false;
    if (!do_topp) return true;
    const uint32_t k = order_key(v);
    return k > kb || (k == kb && idx <= ir);
  };

  // log Z over the kept tokens.
  float zl = 0.f;
  if (!fast) {
    r.pass();
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int idx = r.index(g, e);
        const float v = r.val(8 * g + e);
        if (keep(idx, v)) zl += expf(v - m);
      }
  }
  const float logz = fast ? 0.f : logf(block_sum_f32(zl, sh));

  int tok = amax;
  if (!greedy) {
    u64 local = 0;
    r.pass();
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int idx = r.index(g, e);
        const float v = r.val(8 * g + e);
        if (keep(idx, v)) local += mass_of(v, m);
      }
    const u64 wtot = block_sum_u64(local, sh);
    const u64 target = __umul64hi(draw_u64(a.seed, a.offset, (u64)row), wtot);
    tok = find_first_exceeding(sh, r, target, [&](int idx, float v) { return keep(idx, v) ? mass_of(v, m) : (u64)0; });
  }

  // Outputs: the token (and its log-probability) from the thread holding it,
  // the full log-probabilities of the filtered logits from every thread.
  if ((int)threadIdx.x == ((tok >> 3) & (kThreads - 1))) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (r.index(g, e) == tok) {
          a.tokens[row] = tok;
          if (a.token_logprob) a.token_logprob[row] = (r.val(8 * g + e) - m) - logz;
        }
  }
  if (a.logprobs) {
    r.pass();
    float *dst_row = a.logprobs + (int64_t)row * a.ld_lp;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int base = r.index(g, 0);
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = r.val(8 * g + e);
        o[e] = keep(base + e, v) ? (v - m) - logz : -INFINITY;
      }
      if (a.vec_out && base + 8 <= a.V) {
        *reinterpret_cast<f32x4 *>(dst_row + base) = f32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<f32x4 *>(dst_row + base + 4) = f32x4{o[4], o[5], o[6], o[7]};
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (base + e < a.V) dst_row[base + e] = o[e];
      }
    }
  }
}

// top_k == 1 without the full log-probability rows: the first maximum and
// its log-probability -log(r), r the tied maxima top-p keeps (one, or all of
// them without top-p), exactly what sample_kernel computes for this case; a
// kernel of its own so that the engine's greedy step runs only this code.
template <int EPT, bool kF32>
__global__ __launch_bounds__(kThreads) void greedy_kernel(SampleArgs a) {
  __shared__ SampleShared sh;
  const int row = blockIdx.x;
  Row<EPT, kF32> r;
  load_row<EPT, kF32>(a, row, r);
  const RowMax mx = row_max<EPT, kF32>(a, r, sh);
  if (threadIdx.x == 0) {
    a.tokens[row] = mx.amax;
    if (a.token_logprob) {
      u64 kept = (u64)mx.cmax;
      if (a.apply_top_p) {  // equal masses 2^40: the first max(1, floor(p * c)) ties stay
        const u64 t = (u64)((double)a.top_p * (double)(kept << 40));
        kept = (t >> 40) > 0 ? (t >> 40) : 1;
      }
      a.token_logprob[row] = 0.f - logf((float)kept);
    }
  }
}

template <int EPT, bool kF32>
hipError_t launch_ept(SampleArgs a, hipStream_t s) {
  if (a.top_k == 1 && a.logprobs == nullptr) {
    hipLaunchKernelGGL((greedy_kernel<EPT, kF32>), dim3(a.M), dim3(kThreads), 0, s, a);
    return hipGetLastError();
  }
  if (a.cand != nullptr && a.cand_chunks == sample_cand_chunks(a.M, a.V, a.top_k, a.logprobs != nullptr) &&
      a.cand_chunks > 0) {
    // rows in grid y: sample_cand_chunks is 0 past kMaxCandRows rows
    hipLaunchKernelGGL((topk_candidates_kernel<kF32>), dim3(a.cand_chunks, a.M), dim3(kCandThreads), 0, s, a);
    // sample_kernel must not read candidate records this call did not write
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  } else {
    a.cand = nullptr;
  }
  hipLaunchKernelGGL((sample_kernel<EPT, kF32>), dim3(a.M), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace

int sample_cand_chunks(int64_t rows, int64_t vocab, int64_t top_k, bool logprobs_rows) {
  if (logprobs_rows || top_k < 2 || top_k > kCandSlots || vocab <= kCandChunk || rows > kMaxCandRows) return 0;
  return (int)((vocab + kCandChunk - 1) / kCandChunk);
}

// Rows up to 65536 (bf16) / 32768 (fp32) values: fp32 rows of 64 values per
// thread would not fit in the registers of a 1024-thread workgroup.
hipError_t launch_sample(const SampleArgs &a, bool f32, hipStream_t stream) {
  if (a.M == 0) return hipSuccess;
  if (f32) {
    if (a.V > kMaxSampleVocabF32) return hipErrorInvalidValue;
    if (a.V <= 8 * kThreads) return launch_ept<8, true>(a, stream);
    if (a.V <= 16 * kThreads) return launch_ept<16, true>(a, stream);
    return launch_ept<32, true>(a, stream);
  }
  if (a.V > kMaxSampleVocabBF16) return hipErrorInvalidValue;
  if (a.V <= 8 * kThreads) return launch_ept<8, false>(a, stream);
  if (a.V <= 16 * kThreads) return launch_ept<16, false>(a, stream);
  if (a.V <= 32 * kThreads) return launch_ept<32, false>(a, stream);
  return launch_ept<64, false>(a, stream);
}

}  // namespace tt
