// Decode-step layer kernels for gfx950: the dense work around the attention
// path of one decode step (one token per sequence, M = batch rows).
//
//   skinny GEMM   P[s][m][n] = sum_{k in chunk s} x[m][k] * W[n][k]
//                 (nn.Linear without bias, weights [N, K] bf16; the reference's
//                 projections attn.py:141-145, mlp.py:24-26, gpt.py:62-63)
//   reductions    the split-K partials are summed in a fixed order by the
//                 kernel that consumes them, so results do not depend on
//                 scheduling:
//     reduce_bf16   y = bf16(sum_s P[s])                    (q/k/v projection)
//     add_rmsnorm   x += bf16(sum_s P[s]); y = bf16(w * x * rsqrt(mean(x^2) + eps))
//                   (residual add gpt.py:40-41 + RMSNorm norm.py:6-19)
//     silu_mul      y = bf16(bf16(silu(bf16(sum_s P_gate))) * bf16(sum_s P_up))
//                   (SwiGLU, mlp.py:44-45, with the bf16 rounding points of
//                   the reference under autocast)
//
// The GEMM is weight-bandwidth bound (M <= 64 rows against K x N weights), so
// it is organised around streaming W exactly once, spread over every CU (a
// CU alone draws only a few tens of GB/s): a workgroup owns 64 or 128 output
// columns and one KC-wide chunk of K; each of its waves loads its 16 weight
// rows x KC columns in one burst (all loads in flight together), while the
// workgroup stages the x chunk (64 rows x KC) in LDS. The product runs on
// v_mfma_f32_16x16x32_bf16 with W as the A operand (16 rows = output
// columns) and x^T as the B operand (16 columns = batch rows).
#include <algorithm>

#include "tt_internal.h"
#include "tt_numerics.h"
#include "wave_reduce.h"

namespace tt {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Weight fragment of k step s of 16-row block nb, starting at column k (a
// multiple of 32): lane (i + 16g) reads W[16 nb + i][k + 32 s + 8 g .. + 8].
// Row-major weights: base + 32 s. Packed weights ([N/16][K/32][64 lanes][8],
// the fragment order) make every k step one contiguous 1 KB: base + 512 s.
__device__ __forceinline__ const uint16_t *wfrag_base(const SkinnyGemmArgs &a, int nb, int64_t k, int lane,
                                                      int &step) {
  if (a.packed) {
    step = 512;
    return a.w + (((int64_t)nb * (a.K / 32) + k / 32) * 64 + lane) * 8;
  }
  step = 32;
  return a.w + (int64_t)(nb * 16 + (lane & 15)) * a.ldw + k + 8 * (lane >> 4);
}

// Workgroups of this shape meant to share a CU (bounded by the x chunk's LDS
// footprint, 64 x (KC + 8) x 2 bytes), and the waves per SIMD the register
// allocation must leave room for so that they can.
constexpr int gemm_wgs_per_cu(int kc, int waves) {
  return kc == 256 ? (waves <= 4 ? 4 : waves <= 8 ? 2 : 1) : kc == 512 ? (waves <= 8 ? 2 : 1) : 1;
}

template <int KC, int WAVES>
constexpr int gemm_min_waves() {
  const int w = (WAVES * gemm_wgs_per_cu(KC, WAVES) + 3) / 4;
  return w < 1 ? 1 : w > 4 ? 4 : w;
}

template <int KC, int WAVES>
__global__ __launch_bounds__(64 * WAVES, (gemm_min_waves<KC, WAVES>())) void skinny_gemm_kernel(SkinnyGemmArgs a) {
  constexpr int KSTEPS = KC / 32;
  constexpr int ROW = KC + 8;  // padded LDS row (elements): 16 consecutive rows hit distinct banks
  __shared__ __attribute__((aligned(16))) uint16_t xs[64 * ROW];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * (16 * WAVES) + wave * 16;
  const int64_t k0 = (int64_t)blockIdx.y * KC;
  const int m0 = blockIdx.z * 64;

  // x rows m0 .. m0 + 63 of the chunk (L2-resident, rows past M are zero)
  // are loaded before the weights: vector loads return in issue order, so
  // x issued first can go to LDS while the weight stream is still in flight.
  constexpr int XN = 64 * (KC / 8);                        // 16-byte pieces of the x chunk
  constexpr int XL = (XN + 64 * WAVES - 1) / (64 * WAVES);  // per thread
  u32x4 xr[XL];
#pragma unroll
  for (int j = 0; j < XL; ++j) {
    const int i = threadIdx.x + j * 64 * WAVES;
    const int r = i / (KC / 8);
    const int c = i - r * (KC / 8);
    xr[j] = u32x4{0u, 0u, 0u, 0u};
    if ((XN % (64 * WAVES) == 0 || i < XN) && m0 + r < a.M)
      xr[j] = *reinterpret_cast<const u32x4 *>(a.x + (int64_t)(m0 + r) * a.ldx + k0 + 8 * c);
  }

  // This wave's weight fragments for the whole chunk: lane (i + 16g) holds
  // W[n0 + i][k0 + 32 s + 8 g .. + 8] for k step s.
  int wstep;
  const uint16_t *wrow = wfrag_base(a, n0 / 16, k0, lane, wstep);
  u32x4 wf[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) wf[s] = *reinterpret_cast<const u32x4 *>(wrow + wstep * s);

#pragma unroll
  for (int j = 0; j < XL; ++j) {
    const int i = threadIdx.x + j * 64 * WAVES;
    const int r = i / (KC / 8);
    const int c = i - r * (KC / 8);
    if (XN % (64 * WAVES) == 0 || i < XN) *reinterpret_cast<u32x4 *>(xs + r * ROW + 8 * c) = xr[j];
  }
  __syncthreads();

  f32x4 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    const bf16x8 af = __builtin_bit_cast(bf16x8, wf[s]);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const bf16x8 bfr =
          *reinterpret_cast<const bf16x8 *>(xs + (mb * 16 + (lane & 15)) * ROW + 32 * s + 8 * (lane >> 4));
      acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr, acc[mb], 0, 0, 0);
    }
  }

  // acc[mb]: lane (j + 16g) holds out column n0 + 4g + r (r = 0..3) of batch row m0 + 16 mb + j.
  float *P = a.part + (int64_t)blockIdx.y * a.M * a.N;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int m = m0 + mb * 16 + (lane & 15);
    if (m < a.M) *reinterpret_cast<f32x4 *>(P + (int64_t)m * a.N + n0 + 4 * (lane >> 4)) = acc[mb];
  }
}

// sum_{s < S} P[s * stride + i] added in order s = 0, 1, ..., for n rows i[r]
// at once: the splits go in batches of four whose loads (addresses clamped to
// a valid split, so no branch separates them) are all issued before the
// batch's adds, so S <= 4 costs one memory round trip for every row together.
// Additions past S are selected away; the order of the additions is s = 0,
// 1, ..., S - 1.
template <int n>
__device__ __forceinline__ void ordered_sums(const float *P, int S, int64_t stride, const int64_t (&i)[n],
                                             f32x4 (&d)[n]) {
  for (int s0 = 0; s0 < S; s0 += 4) {
    f32x4 v[n][4];
#pragma unroll
    for (int r = 0; r < n; ++r)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int s = s0 + u < S ? s0 + u : S - 1;
        v[r][u] = *reinterpret_cast<const f32x4 *>(P + (int64_t)s * stride + i[r]);
      }
#pragma unroll
    for (int r = 0; r < n; ++r)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (s0 + u == 0)
          d[r] = v[r][0];
        else
          d[r] = s0 + u < S ? d[r] + v[r][u] : d[r];
      }
  }
}

// y[i] = bf16(sum_s P[s][i]), four elements per thread.
__global__ __launch_bounds__(256) void reduce_bf16_kernel(const float *P, int S, int64_t MN, uint16_t *y) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= MN) return;
  const int64_t ix[1] = {i};
  f32x4 sum[1];
  ordered_sums<1>(P, S, MN, ix, sum);
  const f32x4 acc = sum[0];
  uint32_t lo = pack_bf16x2(acc[0], acc[1]);
  uint32_t hi = pack_bf16x2(acc[2], acc[3]);
  *reinterpret_cast<uint2 *>(y + i) = make_uint2(lo, hi);
}

__device__ __forceinline__ float block_sum_256(float v, float *red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float t = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return t;
}

// One workgroup per row m. With P != null the residual row first takes the
// bf16-rounded sum of the partials (the projection's autocast output). Every
// load of the row (x, up to SMAX splits and the norm weight) is issued before
// the first add, so the row costs one memory round trip; the splits are added
// in order. (Loaded after the block reduction, the weight cost two more round
// trips: the compiler keeps loads below a barrier where the source puts them.)
// PER float4 groups per thread (C <= 1024 * PER, C a multiple of 4; with
// kMask, groups past C are neither loaded nor stored and add 0 to the sum of
// squares; without it C == 1024 * PER and every load is unconditional, so
// all of them go out before the first add); SMAX splits loaded at once
template <int PER, int SMAX, bool kMask>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(float *x, const float *P, int S, int64_t MN,
                                                          const float *w, float eps, uint16_t *y, int C) {
  __shared__ float red[4];
  const int64_t row = (int64_t)blockIdx.x * C;
  f32x4 v[PER], wv[PER];
  f32x4 pv[PER][SMAX];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = 4 * (threadIdx.x + 256 * j);
    const bool in = !kMask || c < C;
    v[j] = in ? *reinterpret_cast<const f32x4 *>(x + row + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    if (P != nullptr) {
#pragma unroll
      for (int s = 0; s < SMAX; ++s)  // splits past S reload split 0 and are not added
        pv[j][s] = in ? *reinterpret_cast<const f32x4 *>(P + (int64_t)(s < S ? s : 0) * MN + row + c)
                      : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {  // issued after the row's loads, which are needed first
    const int c = 4 * (threadIdx.x + 256 * j);
    wv[j] = !kMask || c < C ? *reinterpret_cast<const f32x4 *>(w + c) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = 4 * (threadIdx.x + 256 * j);
    if (kMask && c >= C) continue;
    if (P != nullptr) {
      f32x4 d = pv[j][0];
#pragma unroll
      for (int s = 1; s < SMAX; ++s)
        if (s < S) d += pv[j][s];
      for (int s = SMAX; s < S; ++s) d += *reinterpret_cast<const f32x4 *>(P + (int64_t)s * MN + row + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[j][e] += round_bf16(d[e]);
      *reinterpret_cast<f32x4 *>(x + row + c) = v[j];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += v[j][e] * v[j][e];
  }
  const float var = block_sum_256(ss, red) / (float)C;
  const float r = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = 4 * (threadIdx.x + 256 * j);
    if (kMask && c >= C) continue;
    uint32_t lo = pack_bf16x2(wv[j][0] * (v[j][0] * r), wv[j][1] * (v[j][1] * r));
    uint32_t hi = pack_bf16x2(wv[j][2] * (v[j][2] * r), wv[j][3] * (v[j][3] * r));
    *reinterpret_cast<uint2 *>(y + row + c) = make_uint2(lo, hi);
  }
}

// SwiGLU with the reference's autocast rounding points (mlp.py:44-45): the
// projections return bf16, F.silu runs in bf16, the product rounds to bf16.
__device__ __forceinline__ uint16_t swiglu_bf16(float g, float u) {
  const float gb = round_bf16(g);
  const float act = round_bf16(gb / (1.0f + expf(-gb)));
  return f32_to_bf16_bits(act * round_bf16(u));
}

// Partials of the fused gate|up projection: columns [0, I) gate, [I, 2I) up.
__global__ __launch_bounds__(256) void silu_mul_kernel(const float *P, int S, int64_t MN2, int I, int M,
                                                       uint16_t *y) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;  // index into [M, I]
  if (i >= (int64_t)M * I) return;
  const int64_t m = i / I;
  const int64_t c = i - m * I;
  const int64_t gi = m * 2 * I + c;
  const int64_t ix[2] = {gi, gi + I};
  f32x4 sum[2];
  ordered_sums<2>(P, S, MN2, ix, sum);
  const f32x4 g = sum[0];
  const f32x4 u = sum[1];
  uint16_t out[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = swiglu_bf16(g[e], u[e]);
  *reinterpret_cast<uint2 *>(y + i) = make_uint2(out[0] | ((uint32_t)out[1] << 16), out[2] | ((uint32_t)out[3] << 16));
}

// Gate|up projection with SwiGLU in the epilogue (mlp.py:24-26, 44-45):
// a[m][c] = swiglu(x[m] . Wg[c], x[m] . Wu[c]) over the whole K inside one
// workgroup, so no split-K partials and no second launch. The weight is the
// fragment-ordered [gate|up] matrix with its rows interleaved by 8: 16-row
// block j holds gate rows 8j .. 8j+7, then up rows 8j .. 8j+7, so the MFMA
// output puts gate row r of a block in lane (n + 16g), g < 2, and up row r in
// lane (n + 16g) ^ 32.
//
// A workgroup owns NB 16-row blocks (8 NB output columns) and 2 NB waves:
// wave (block, half) streams its 16 rows x K/2 (one
// burst, 128 registers at K = 2048). The x rows (64 per m tile) reach LDS by
// DMA (buffer_load ... lds, one 1 KiB row chunk per instruction, rows past M
// read as zero) in two rounds of K/4 columns per half, the first issued
// before the weight burst, the second after the first round's MFMAs (its
// loads retire after the weights, which they queue behind). The two halves
// of a block meet in LDS (sum half 0 + half 1), then the gate lanes exchange
// with the up lanes and write 4 bf16 outputs each.
// K = 1024 R (R = 1, 2): R staging rounds, each one 512-column (1 KiB) row
// chunk per half, so the LDS holds one round (133 KB, one workgroup per CU)
// whatever K. K = 768: one round of 384 columns per half, staged by the same
// 1 KiB row chunks (the 128 columns past a half are loaded and not used; past
// the last row's end the buffer bound reads zero). NB = 2, 3 or 4 row blocks
// per workgroup (the launcher picks one
// that divides I / 8: 3 where it can, the measured layout).
// (Register budget: two workgroups' worth per CU, as measured for NB = 3;
// NB = 4 with 128 weight registers per lane fits one.)
template <int K, int NB>
__global__ __launch_bounds__(64 * 2 * NB, NB == 4 ? 1 : 2) void swiglu_gemm_kernel(SwigluGemmArgs a) {
  constexpr int R = (K + 1023) / 1024; // staging rounds
  constexpr int KS = K / 64;           // k steps per wave (its half of K)
  constexpr int KQ = K / (2 * R);      // columns per half per round (512; 384 at K = 768)
  constexpr int ROW = 512 + 8;         // padded LDS row (elements): one 1 KiB DMA chunk
  static_assert((K == 768 || K == 1024 || K == 2048) && KQ <= 512 && KS <= 32, "K = 768, 1024 or 2048");
  constexpr int kWaves = 2 * NB;
  constexpr int kRows = 2 * 64;        // LDS rows per round: 2 halves x 64 x rows
  __shared__ __attribute__((aligned(16))) uint16_t xs[kRows * ROW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = wave >> 1;           // row block of this workgroup
  const int half = wave & 1;           // K half
  const int nb = blockIdx.x * NB + blk;
  const int m0 = blockIdx.z * 64;
  const int mrows = min(64, a.M - m0);

  // x rows m0 .. m0 + mrows - 1; offsets past the last valid row's data read zero
  const auto rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.x) + (int64_t)m0 * a.ldx, (short)0,
      (int)(((int64_t)(mrows - 1) * a.ldx + K) * 2), 0x00020000);
  auto stage = [&](int round) {
    for (int i = wave; i < kRows; i += kWaves) {  // i = h * 64 + row
      const int h = i >> 6, r = i & 63;
      const int col = h * (K / 2) + round * KQ;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void *)(xs + i * ROW), 16,
                                               16 * lane + (int)(((int64_t)r * a.ldx + col) * 2), 0, 0, 0);
    }
  };

  stage(0);
  __builtin_amdgcn_sched_barrier(0);
  const uint16_t *wrow = a.w + (((int64_t)nb * (K / 32) + half * KS) * 64 + lane) * 8;
  u32x4 wf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {  // in consumption order: each k step waits only for its own loads
    wf[s] = *reinterpret_cast<const u32x4 *>(wrow + 512 * s);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_waitcnt((KS & 15) | (7 << 4) | (15 << 8) | (((KS >> 4) & 3) << 14));  // this wave's x DMA
  __syncthreads();

  f32x4 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint16_t *xrow = xs + (half * 64 + (lane & 15)) * ROW + 8 * (lane >> 4);
#pragma unroll
  for (int round = 0; round < R; ++round) {
    if (round > 0) {
      __syncthreads();  // every wave is done with the previous round's x
      stage(round);
      __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));
      __syncthreads();
    }
#pragma unroll
    for (int s = 0; s < KS / R; ++s) {
      const bf16x8 af = __builtin_bit_cast(bf16x8, wf[round * (KS / R) + s]);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16x8 bfr = *reinterpret_cast<const bf16x8 *>(xrow + mb * 16 * ROW + 32 * s);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr, acc[mb], 0, 0, 0);
      }
    }
  }

  // the halves meet: half 0 finishes m blocks 0-1, half 1 blocks 2-3
  __syncthreads();
  f32x4 *red = reinterpret_cast<f32x4 *>(xs);  // [block][half][2][64]
#pragma unroll
  for (int j = 0; j < 2; ++j) red[((blk * 2 + half) * 2 + j) * 64 + lane] = acc[half == 0 ? 2 + j : j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int mb = half == 0 ? j : 2 + j;
    const f32x4 other = red[((blk * 2 + (1 - half)) * 2 + j) * 64 + lane];
    const f32x4 sum = half == 0 ? acc[mb] + other : other + acc[mb];
    f32x4 up;
#pragma unroll
    for (int r = 0; r < 4; ++r) up[r] = __shfl_xor(sum[r], 32, 64);
    const int row = 16 * mb + (lane & 15);
    if (lane < 32 && row < mrows) {
      uint16_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = swiglu_bf16(sum[r], up[r]);
      *reinterpret_cast<uint2 *>(a.out + (int64_t)(m0 + row) * a.ldo + 8 * nb + 4 * (lane >> 4)) =
          make_uint2(o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16));
    }
  }
}

// Prefill rows (many tokens, bf16 projection outputs from a library GEMM):
// x += float(a[m]) (a: bf16 [M, C] with row stride lda, the projection's
// autocast output; a == nullptr skips the add), then
// y = bf16(w * x * rsqrt(mean(x^2) + eps)) as in add_rmsnorm_kernel.
template <int PER, bool kMask>  // as add_rmsnorm_kernel
__global__ __launch_bounds__(256) void add_rmsnorm_rows_kernel(float *x, const uint16_t *a, int64_t lda,
                                                               const float *w, float eps, uint16_t *y, int C) {
  __shared__ float red[4];
  const int64_t row = (int64_t)blockIdx.x * C;
  f32x4 v[PER], wv[PER];
  uint2 av[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = 4 * (threadIdx.x + 256 * j);
    const bool in = !kMask || c < C;
    v[j] = in ? *reinterpret_cast<const f32x4 *>(x + row + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    av[j] = make_uint2(0u, 0u);
    if (a != nullptr && in) av[j] = *reinterpret_cast<const uint2 *>(a + (int64_t)blockIdx.x * lda + c);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {  // the weight with the row's loads: one round trip
    const int c = 4 * (threadIdx.x + 256 * j);
    wv[j] = !kMask || c < C ? *reinterpret_cast<const f32x4 *>(w + c) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (kMask && 4 * (threadIdx.x + 256 * j) >= C) continue;
    if (a != nullptr) {
      v[j][0] += __builtin_bit_cast(float, av[j].x << 16);
      v[j][1] += __builtin_bit_cast(float, av[j].x & 0xffff0000u);
      v[j][2] += __builtin_bit_cast(float, av[j].y << 16);
      v[j][3] += __builtin_bit_cast(float, av[j].y & 0xffff0000u);
      *reinterpret_cast<f32x4 *>(x + row + 4 * (threadIdx.x + 256 * j)) = v[j];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += v[j][e] * v[j][e];
  }
  const float var = block_sum_256(ss, red) / (float)C;
  const float r = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = 4 * (threadIdx.x + 256 * j);
    if (kMask && c >= C) continue;
    uint32_t lo = pack_bf16x2(wv[j][0] * (v[j][0] * r), wv[j][1] * (v[j][1] * r));
    uint32_t hi = pack_bf16x2(wv[j][2] * (v[j][2] * r), wv[j][3] * (v[j][3] * r));
    *reinterpret_cast<uint2 *>(y + row + c) = make_uint2(lo, hi);
  }
}

// SwiGLU of bf16 gate and up projection outputs (rows m of g and u, row
// strides ldg / ldu): y[m][i] = bf16(bf16(silu(g)) * u), y contiguous
// [M, I]; four columns per thread.
__global__ __launch_bounds__(256) void silu_mul_rows_kernel(const uint16_t *g_in, int64_t ldg, const uint16_t *u_in,
                                                            int64_t ldu, int I, int64_t MI, uint16_t *y) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;  // index into [M, I]
  if (i >= MI) return;
  const int64_t m = i / I;
  const int64_t c = i - m * I;
  const uint2 g2 = *reinterpret_cast<const uint2 *>(g_in + m * ldg + c);
  const uint2 u2 = *reinterpret_cast<const uint2 *>(u_in + m * ldu + c);
  const float g[4] = {__builtin_bit_cast(float, g2.x << 16), __builtin_bit_cast(float, g2.x & 0xffff0000u),
                      __builtin_bit_cast(float, g2.y << 16), __builtin_bit_cast(float, g2.y & 0xffff0000u)};
  const float u[4] = {__builtin_bit_cast(float, u2.x << 16), __builtin_bit_cast(float, u2.x & 0xffff0000u),
                      __builtin_bit_cast(float, u2.y << 16), __builtin_bit_cast(float, u2.y & 0xffff0000u)};
  uint16_t out[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float act = round_bf16(g[e] / (1.0f + expf(-g[e])));
    out[e] = f32_to_bf16_bits(act * u[e]);
  }
  *reinterpret_cast<uint2 *>(y + i) = make_uint2(out[0] | ((uint32_t)out[1] << 16), out[2] | ((uint32_t)out[3] << 16));
}

}  // namespace

hipError_t launch_skinny_gemm(const SkinnyGemmArgs &a, int kc, hipStream_t stream) {
  const int cus = device_cu_count();
  const int splits = a.K / kc, mt = (a.M + 63) / 64;
  int waves;
  if (kc == 1024) {
    // One workgroup per CU (the x chunk takes 132 KB of LDS): the shape whose
    // busiest CU streams the fewest weight rows. (gate|up at C5, N 12288 on
    // 256 CUs: 6 waves, one 192 KB workgroup per CU, 14.7-15.1 us against
    // 16.1-16.5 us for 8-wave workgroups at 512-wide chunks.)
    waves = 4;
    int64_t best = -1;
    for (int w : {4, 6, 8}) {
      if (a.N % (16 * w)) continue;
      const int64_t wgs = (int64_t)(a.N / (16 * w)) * splits * mt;
      const int64_t rows = (wgs + cus - 1) / cus * w;
      if (best < 0 || rows < best) {
        best = rows;
        waves = w;
      }
    }
  } else {
    // 8 waves (128 weight rows) share one staged x chunk when that still puts
    // a workgroup on at least 3/4 of the CUs; otherwise 4 waves (64 rows).
    // (Measured on the decode-step shapes: two 8-wave workgroups on some CUs
    // beat one 12-wave workgroup on every CU; 6- and 12-wave groups lost.)
    const bool wide = a.N % 128 == 0 && 4 * (int64_t)(a.N / 128) * splits * mt >= 3 * (int64_t)cus;
    waves = wide ? 8 : 4;
  }
  const dim3 grid((unsigned)(a.N / (16 * waves)), (unsigned)splits, (unsigned)mt);
#define TT_GEMM_LAUNCH(KC, W) hipLaunchKernelGGL((skinny_gemm_kernel<KC, W>), grid, dim3(64 * W), 0, stream, a)
  if (kc == 256) {
    if (waves == 8) TT_GEMM_LAUNCH(256, 8); else TT_GEMM_LAUNCH(256, 4);
  } else if (kc == 512) {
    if (waves == 8) TT_GEMM_LAUNCH(512, 8); else TT_GEMM_LAUNCH(512, 4);
  } else {
    if (waves == 8) TT_GEMM_LAUNCH(1024, 8); else if (waves == 6) TT_GEMM_LAUNCH(1024, 6); else TT_GEMM_LAUNCH(1024, 4);
  }
#undef TT_GEMM_LAUNCH
  return hipGetLastError();
}

hipError_t launch_reduce_bf16(const float *P, int S, int64_t MN, uint16_t *y, hipStream_t stream) {
  const int64_t threads = (MN + 3) / 4;
  hipLaunchKernelGGL(reduce_bf16_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, P, S, MN, y);
  return hipGetLastError();
}

hipError_t launch_add_rmsnorm(float *x, const float *P, int S, int M, int C, const float *w, float eps, uint16_t *y,
                              hipStream_t stream) {
  const int64_t MN = (int64_t)M * C;
#define TT_ADD_RMSNORM_LAUNCH(n, smax)                                                                       \
  do {                                                                                                      \
    if (C % 1024 == 0)                                                                                      \
      hipLaunchKernelGGL((add_rmsnorm_kernel<n, smax, false>), dim3(M), dim3(256), 0, stream, x, P, S, MN, w, eps, \
                         y, C);                                                                             \
    else                                                                                                    \
      hipLaunchKernelGGL((add_rmsnorm_kernel<n, smax, true>), dim3(M), dim3(256), 0, stream, x, P, S, MN, w, eps, \
                         y, C);                                                                             \
  } while (0)
#define TT_ADD_RMSNORM_CASE(n)                  \
  case n:                                       \
    if (S <= 4)                                 \
      TT_ADD_RMSNORM_LAUNCH(n, 4);              \
    else if (S <= 8 && n <= 4)                  \
      TT_ADD_RMSNORM_LAUNCH(n, (n <= 4 ? 8 : 4)); \
    else                                        \
      TT_ADD_RMSNORM_LAUNCH(n, (n <= 2 ? 16 : 4)); \
    break;
  switch ((C + 1023) / 1024) {  // C a multiple of 4 in [4, 8192], checked by the caller
    TT_ADD_RMSNORM_CASE(1)
    TT_ADD_RMSNORM_CASE(2)
    TT_ADD_RMSNORM_CASE(3)
    TT_ADD_RMSNORM_CASE(4)
    TT_ADD_RMSNORM_CASE(5)
    TT_ADD_RMSNORM_CASE(6)
    TT_ADD_RMSNORM_CASE(7)
    TT_ADD_RMSNORM_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef TT_ADD_RMSNORM_CASE
#undef TT_ADD_RMSNORM_LAUNCH
  return hipGetLastError();
}

bool swiglu_gemm_supported(int64_t K, int64_t I) {
  return (K == 768 || K == 1024 || K == 2048) && I > 0 && (I % 24 == 0 || I % 16 == 0);
}

// Row blocks per workgroup for intermediate size I: 3 (the measured layout)
// when 24 divides I, else 4 while that still gives every CU a workgroup, else 2.
int swiglu_row_blocks(int64_t I) {
  if (I % 24 == 0) return 3;
  if (I % 32 == 0 && I / 32 >= device_cu_count()) return 4;
  return 2;
}

template <int K>
hipError_t launch_swiglu_k(const SwigluGemmArgs &a, hipStream_t stream) {
  const int nb = swiglu_row_blocks(a.I);
  const dim3 grid((unsigned)(a.I / (8 * nb)), 1, (unsigned)((a.M + 63) / 64));
  if (nb == 3)
    hipLaunchKernelGGL((swiglu_gemm_kernel<K, 3>), grid, dim3(128 * 3), 0, stream, a);
  else if (nb == 4)
    hipLaunchKernelGGL((swiglu_gemm_kernel<K, 4>), grid, dim3(128 * 4), 0, stream, a);
  else
    hipLaunchKernelGGL((swiglu_gemm_kernel<K, 2>), grid, dim3(128 * 2), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_swiglu_gemm(const SwigluGemmArgs &a, hipStream_t stream) {
  if (a.K == 768) return launch_swiglu_k<768>(a, stream);
  if (a.K == 1024) return launch_swiglu_k<1024>(a, stream);
  if (a.K == 2048) return launch_swiglu_k<2048>(a, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_silu_mul(const float *P, int S, int M, int I, uint16_t *y, hipStream_t stream) {
  const int64_t threads = ((int64_t)M * I + 3) / 4;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, P, S,
                     (int64_t)M * 2 * I, I, M, y);
  return hipGetLastError();
}

hipError_t launch_add_rmsnorm_rows(float *x, const uint16_t *a, int64_t lda, int M, int C, const float *w, float eps,
                                   uint16_t *y, hipStream_t stream) {
  switch ((C + 1023) / 1024) {  // C a multiple of 4 in [4, 8192], checked by the caller
#define TT_ROWS_CASE(n)                                                                                              \
  case n:                                                                                                            \
    if (C % 1024 == 0)                                                                                               \
      hipLaunchKernelGGL((add_rmsnorm_rows_kernel<n, false>), dim3(M), dim3(256), 0, stream, x, a, lda, w, eps, y, C); \
    else                                                                                                             \
      hipLaunchKernelGGL((add_rmsnorm_rows_kernel<n, true>), dim3(M), dim3(256), 0, stream, x, a, lda, w, eps, y, C); \
    break;
    TT_ROWS_CASE(1)
    TT_ROWS_CASE(2)
    TT_ROWS_CASE(3)
    TT_ROWS_CASE(4)
    TT_ROWS_CASE(5)
    TT_ROWS_CASE(6)
    TT_ROWS_CASE(7)
    TT_ROWS_CASE(8)
#undef TT_ROWS_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_silu_mul_rows(const uint16_t *g, int64_t ldg, const uint16_t *u, int64_t ldu, int64_t M, int I,
                                uint16_t *y, hipStream_t stream) {
  const int64_t threads = (M * I + 3) / 4;
  hipLaunchKernelGGL(silu_mul_rows_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, g, ldg, u,
                     ldu, I, M * I, y);
  return hipGetLastError();
}

}  // namespace tt
