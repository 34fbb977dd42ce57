// Fused RoPE + KV-cache append for gfx950.
//
// One 64-lane wave per (row, new token, sequence), where rows 0..H_q-1 are
// query heads (rotated into q_out) and rows H_q..H_q+H_kv-1 are KV heads
// (K rotated, V copied, both written into the cache slot of the token).
// Lane i < D/2 owns the rotation pair (x_i, x_{i+D/2}), which is the pair
// rotate_half mixes (attn.py:56-59), so the wave holds a whole head row and
// the fp8 absmax is a single wave reduction.
//
// The work is a few hundred KB per decode step and is latency bound; its
// role is to produce bytes identical to the reference's rope_impl
// (attn.py:13-63) and cache append (cache.py:41-42) at the slot given by the
// per-sequence position.
#include "rope_math.h"
#include "tt_internal.h"
#include "tt_numerics.h"
#include "wave_reduce.h"

namespace tt {
namespace {

// Slot element offset of token `pos` of sequence b, KV head hk; -1 if the
// slot is outside the cache (capacity, page table or pool).
__device__ __forceinline__ int64_t slot_offset(const RopeAppendArgs &a, int b, int hk, int64_t pos) {
  if (pos < 0 || pos >= a.capacity) return -1;
  const int64_t j = pos / a.page_size;
  const int64_t slot = pos - j * a.page_size;
  int64_t base;
  if (a.page_table != nullptr) {
    if (j >= a.max_pages) return -1;
    const int64_t phys = a.page_table[(int64_t)b * a.max_pages + j];
    if (phys < 0 || phys >= a.num_pages) return -1;
    base = phys * a.c_page;
  } else {
    base = (int64_t)b * a.c_seq + j * a.c_page;
  }
  return base + (int64_t)hk * a.c_head + slot * a.head_dim;
}

// An input element: the activation at p[i] (kPart 0), or with split-K
// partials the activation-typed sum of the splits added in order (the
// projection's output), in batches of four loads (addresses clamped to a
// valid split, additions past S selected away). kPart 1 (at most four
// splits) loads a wave's inputs inline instead, all before the first add.
template <typename A, int kPart>
__device__ __forceinline__ float load_in(const RopeAppendArgs &a, const void *p, int64_t i) {
  if constexpr (kPart == 0) {
    return Elem<A>::load(p, i);
  } else {
    const float *f = static_cast<const float *>(p);
    const int S = a.part_splits;
    float acc = 0.f;
    for (int s0 = 0; s0 < (kPart == 1 ? 1 : S); s0 += 4) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = f[(int64_t)(s0 + u < S ? s0 + u : S - 1) * a.part_stride + i];
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = s0 + u == 0 ? v[0] : (s0 + u < S ? acc + v[u] : acc);
    }
    return Elem<A>::rnd(acc);
  }
}

// The rest of one (row, token) after its inputs and table entries are in:
// the rotated q row to q_out, or the rotated k and v into the token's cache
// slot (fp8: codes and the per-(token, head) scales). `off` is the slot's
// element offset (from the page entry `phys` of the paged pool).
template <typename A, bool kFP8>
__device__ __forceinline__ void finish_token(const RopeAppendArgs &a, int b, int row, int t, int64_t off, bool is_q,
                                             int i, int half, bool active, float x1, float x2, float v1, float v2,
                                             float c, float s) {
  if (is_q) {
    if (!active) return;
    float o1, o2;
    rotate_pair<A>(x1, x2, c, s, o1, o2);
    const int64_t dst = (int64_t)b * a.qo_sb + (int64_t)row * a.qo_sh + (int64_t)t * a.qo_st;
    Elem<A>::store(a.q_out, dst + i, o1);
    Elem<A>::store(a.q_out, dst + half + i, o2);
    return;
  }

  if (off < 0) return;
  float k1 = 0.f, k2 = 0.f;
  if (active) rotate_pair<A>(x1, x2, c, s, k1, k2);

  if constexpr (!kFP8) {
    if (active) {
      Elem<A>::store(a.k_cache, off + i, k1);
      Elem<A>::store(a.k_cache, off + half + i, k2);
      Elem<A>::store(a.v_cache, off + i, v1);
      Elem<A>::store(a.v_cache, off + half + i, v2);
    }
  } else {
    // Per-(token, head) symmetric scale: absmax / 448, codes e4m3fn(x / scale).
    const float kmax = wave_max_nan(absmax2(0.f, k1, k2));
    const float vmax = wave_max_nan(absmax2(0.f, v1, v2));
    const float kscale = kmax / 448.0f;
    const float vscale = vmax / 448.0f;
    if (active) {
      uint8_t *kc = static_cast<uint8_t *>(a.k_cache);
      uint8_t *vc = static_cast<uint8_t *>(a.v_cache);
      kc[off + i] = e4m3_row_code(k1, kscale);
      kc[off + half + i] = e4m3_row_code(k2, kscale);
      vc[off + i] = e4m3_row_code(v1, vscale);
      vc[off + half + i] = e4m3_row_code(v2, vscale);
    }
    if (i == 0) {
      a.k_scale[fp8_scale_index(off / a.head_dim)] = kscale;
      a.v_scale[fp8_scale_index(off / a.head_dim)] = vscale;
    }
  }
}

template <typename A, bool kFP8, int kPart>
__global__ __launch_bounds__(64) void rope_append_kernel(RopeAppendArgs a) {
  const int row = blockIdx.x;
  const int t = blockIdx.y;
  const int b = blockIdx.z;
  const int i = threadIdx.x;
  const int half = a.head_dim >> 1;
  const bool active = i < half;
  const bool is_q = row < a.hq;
  const int hk = row - a.hq;
  // The inputs do not depend on the position: their loads go out first (all
  // of them, then a scheduling barrier, then the sums), so the position ->
  // (table row, page entry) chain overlaps them. Lanes past D/2 load lane
  // i mod D/2 and drop it, which keeps the loads free of branches.
  const int pos0 = a.positions[b];  // issued with the input loads below
  float x1 = 0.f, x2 = 0.f, v1 = 0.f, v2 = 0.f;
  if (t < a.num_new) {
    const int li = i % half;  // lane i < D/2 reads its own pair; lanes past D/2 a valid one they drop
    const void *p1 = is_q ? a.q_in : a.k_in;
    const int64_t o1 = is_q ? (int64_t)b * a.qi_sb + (int64_t)row * a.qi_sh + (int64_t)t * a.qi_st
                            : (int64_t)b * a.ki_sb + (int64_t)hk * a.ki_sh + (int64_t)t * a.ki_st;
    const int64_t o2 = is_q ? o1 : (int64_t)b * a.vi_sb + (int64_t)hk * a.vi_sh + (int64_t)t * a.vi_st;
    const void *p2 = is_q ? a.q_in : a.v_in;  // q rows load their own row twice; the second copy is unused
    if constexpr (kPart == 1) {
      const float *f1 = static_cast<const float *>(p1);
      const float *f2 = static_cast<const float *>(p2);
      const int S = a.part_splits;
      float r[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t so = (int64_t)(u < S ? u : S - 1) * a.part_stride;
        r[0][u] = f1[so + o1 + li];
        r[1][u] = f1[so + o1 + half + li];
        r[2][u] = f2[so + o2 + li];
        r[3][u] = f2[so + o2 + half + li];
      }
      __builtin_amdgcn_sched_barrier(0);
      float acc[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[k] = r[k][0];
#pragma unroll
        for (int u = 1; u < 4; ++u) acc[k] = u < S ? acc[k] + r[k][u] : acc[k];
        acc[k] = Elem<A>::rnd(acc[k]);
      }
      x1 = acc[0];
      x2 = acc[1];
      v1 = acc[2];
      v2 = acc[3];
    } else {
      x1 = load_in<A, kPart>(a, p1, o1 + li);
      x2 = load_in<A, kPart>(a, p1, o1 + half + li);
      if (!is_q) {
        v1 = load_in<A, kPart>(a, p2, o2 + li);
        v2 = load_in<A, kPart>(a, p2, o2 + half + li);
      }
    }
  }
  if (a.lens_out != nullptr && row == 0 && t == 0 && threadIdx.x == 0) {
    const int n = a.new_lens != nullptr ? min(max(a.new_lens[b], 0), a.num_new) : a.num_new;
    a.lens_out[b] = pos0 + n;
  }
  if (t >= a.num_new) return;  // num_new == 0 launches one row only for lens_out
  const int64_t pos = (int64_t)pos0 + t;
  if (pos < 0 || pos >= a.table_len) return;
  float c = 0.f, s = 0.f;
  if (active) {
    c = Elem<A>::load(a.table, pos * a.head_dim + i);
    s = Elem<A>::load(a.table, pos * a.head_dim + half + i);
  }

  if (is_q) {
    finish_token<A, kFP8>(a, b, row, t, 0, true, i, half, active, x1, x2, v1, v2, c, s);
    return;
  }
  if (a.new_lens != nullptr && t >= a.new_lens[b]) return;  // padding token: no cache write
  finish_token<A, kFP8>(a, b, row, t, slot_offset(a, b, hk, pos), false, i, half, active, x1, x2, v1, v2, c, s);
}

// Prompt chunks (num_new > 1, or packed prompt rows; activations as inputs):
// one wave per (row, group of kChunkTok tokens, sequence). Every token's
// inputs, table entries and (KV rows) page entry are loaded before the first
// is used, so a wave costs about one memory round trip for its kChunkTok
// tokens instead of two per token; the per-token arithmetic is
// finish_token's. Groups past a sequence's new tokens exit at once (KV rows
// always, q rows for packed inputs).
constexpr int kChunkTok = 8;

template <typename A, bool kFP8>
__global__ __launch_bounds__(64) void rope_append_chunk_kernel(RopeAppendArgs a) {
  const int row = blockIdx.x;
  const int tb = blockIdx.y * kChunkTok;
  const int b = blockIdx.z;
  const int i = threadIdx.x;
  const int half = a.head_dim >> 1;
  const bool active = i < half;
  const int li = i % half;  // lane i < D/2 reads its own pair; lanes past D/2 a valid one they drop
  const bool is_q = row < a.hq;
  const int hk = row - a.hq;
  const bool packed = a.in_rows != nullptr;
  const int pos0 = a.positions[b];
  const int nlen = a.new_lens != nullptr ? min(max(a.new_lens[b], 0), a.num_new) : a.num_new;
  const int64_t r0 = packed ? a.in_rows[b] : 0;
  if (a.lens_out != nullptr && row == 0 && blockIdx.y == 0 && threadIdx.x == 0) a.lens_out[b] = pos0 + nlen;
  // KV rows write only the new tokens; packed inputs have no padding rows at all
  if (tb >= nlen && (packed || !is_q)) return;  // uniform
  const int tmax = packed ? nlen - 1 : a.num_new - 1;
  const void *p1 = is_q ? a.q_in : a.k_in;
  const int64_t o1 = is_q ? (packed ? 0 : (int64_t)b * a.qi_sb) + (int64_t)row * a.qi_sh
                          : (packed ? 0 : (int64_t)b * a.ki_sb) + (int64_t)hk * a.ki_sh;
  const int64_t st1 = is_q ? a.qi_st : a.ki_st;
  const int64_t o2 = (packed ? 0 : (int64_t)b * a.vi_sb) + (int64_t)hk * a.vi_sh;
  float x1[kChunkTok], x2[kChunkTok], v1[kChunkTok], v2[kChunkTok], c[kChunkTok], sn[kChunkTok];
  int64_t phys[kChunkTok];
#pragma unroll
  for (int u = 0; u < kChunkTok; ++u) {
    const int t = min(tb + u, tmax);
    // input row of token t: packed rows are clamped to the buffer
    const int64_t tr = packed ? max(min(r0 + t, a.num_rows - 1), (int64_t)0) : (int64_t)t;
    const int64_t pos = (int64_t)pos0 + t;
    const int64_t tp = pos < 0 ? 0 : (pos >= a.table_len ? a.table_len - 1 : pos);
    x1[u] = Elem<A>::load(p1, o1 + tr * st1 + li);
    x2[u] = Elem<A>::load(p1, o1 + tr * st1 + half + li);
    v1[u] = is_q ? 0.f : Elem<A>::load(a.v_in, o2 + tr * a.vi_st + li);
    v2[u] = is_q ? 0.f : Elem<A>::load(a.v_in, o2 + tr * a.vi_st + half + li);
    c[u] = Elem<A>::load(a.table, tp * a.head_dim + li);
    sn[u] = Elem<A>::load(a.table, tp * a.head_dim + half + li);
    int64_t j = pos < 0 ? 0 : pos / a.page_size;
    j = j < a.max_pages ? j : a.max_pages - 1;
    phys[u] = (a.page_table != nullptr && !is_q) ? a.page_table[(int64_t)b * a.max_pages + j] : 0;
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < kChunkTok; ++u) {
    const int t = tb + u;
    const int64_t pos = (int64_t)pos0 + t;
    if (t >= a.num_new || pos < 0 || pos >= a.table_len) continue;  // uniform
    if (is_q) {
      if (packed && t >= nlen) continue;  // no such input row
      finish_token<A, kFP8>(a, b, row, t, 0, true, i, half, active, x1[u], x2[u], 0.f, 0.f, c[u], sn[u]);
      continue;
    }
    if (t >= nlen) continue;  // padding token: no cache write
    int64_t off = -1;        // slot_offset, from the page entry loaded above
    if (pos < a.capacity) {
      const int64_t j = pos / a.page_size;
      const int64_t slot = pos - j * a.page_size;
      if (a.page_table == nullptr)
        off = (int64_t)b * a.c_seq + j * a.c_page + (int64_t)hk * a.c_head + slot * a.head_dim;
      else if (j < a.max_pages && phys[u] >= 0 && phys[u] < a.num_pages)
        off = phys[u] * a.c_page + (int64_t)hk * a.c_head + slot * a.head_dim;
    }
    finish_token<A, kFP8>(a, b, row, t, off, false, i, half, active, x1[u], x2[u], v1[u], v2[u], c[u], sn[u]);
  }
}

// Prompt chunks with bf16 activations and a power-of-two head_dim in
// [16, 128]: a lane holds four consecutive rotation pairs (i .. i+3 and
// i+D/2 .. i+D/2+3), D/8 lanes per token, so every input, table and output
// access is 8 bytes wide (the kernel above moves one 2-byte element per
// lane). A wave covers kVecTok tokens in D/16 passes of 512/D tokens, every
// pass's loads (and page entries) issued before the first is used; same
// per-element arithmetic (rotate_pair) and early exits as the kernel above;
// fp8 scales reduce over the token's D/8 lanes. The kernel is bound by
// instruction issue, not bytes: head_dim (kDsh = log2) is a template
// argument and page_size a power of two, so page, slot and scale indices
// are shifts (a 64-bit integer division is a long VALU sequence), and the
// per-wave set-up is spread over 32 tokens.
__device__ __forceinline__ void unpack4(uint2 w, float (&f)[4]) {
  f[0] = __builtin_bit_cast(float, w.x << 16);
  f[1] = __builtin_bit_cast(float, w.x & 0xffff0000u);
  f[2] = __builtin_bit_cast(float, w.y << 16);
  f[3] = __builtin_bit_cast(float, w.y & 0xffff0000u);
}

__device__ __forceinline__ uint2 pack4(const float (&f)[4]) {
  return make_uint2(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]));
}

constexpr int kVecTok = 32;

template <bool kFP8, int kDsh>
__global__ __launch_bounds__(64) void rope_append_vec_kernel(RopeAppendArgs a) {
  static_assert(kDsh >= 4 && kDsh <= 7, "head_dim 16 .. 128");
  constexpr int D = 1 << kDsh;
  constexpr int dsh = kDsh;
  constexpr int half = D >> 1;
  constexpr int lsh = kDsh - 3;           // log2(lanes per token)
  constexpr int lpt = 1 << lsh;
  constexpr int tpp = 64 >> lsh;          // tokens per pass
  constexpr int kPasses = kVecTok / tpp;  // D / 16
  const int row = blockIdx.x;
  const int tb = blockIdx.y * kVecTok;
  const int b = blockIdx.z;
  const int lane = threadIdx.x;
  const int sub = lane >> lsh;  // this lane's token within a pass
  const int e0 = 4 * (lane & (lpt - 1));
  const bool is_q = row < a.hq;
  const int hk = row - a.hq;
  const bool packed = a.in_rows != nullptr;
  const int pos0 = a.positions[b];
  const int nlen = a.new_lens != nullptr ? min(max(a.new_lens[b], 0), a.num_new) : a.num_new;
  const int64_t r0 = packed ? a.in_rows[b] : 0;
  if (a.lens_out != nullptr && row == 0 && blockIdx.y == 0 && threadIdx.x == 0) a.lens_out[b] = pos0 + nlen;
  if (tb >= nlen && (packed || !is_q)) return;  // uniform
  const int tmax = packed ? nlen - 1 : a.num_new - 1;
  const int psh = __builtin_ctz(a.page_size);  // a power of two (vec_ok)
  const uint16_t *p1 = static_cast<const uint16_t *>(is_q ? a.q_in : a.k_in);
  const uint16_t *pv = static_cast<const uint16_t *>(a.v_in);
  const uint16_t *tab = static_cast<const uint16_t *>(a.table);
  const int64_t o1 = is_q ? (packed ? 0 : (int64_t)b * a.qi_sb) + (int64_t)row * a.qi_sh
                          : (packed ? 0 : (int64_t)b * a.ki_sb) + (int64_t)hk * a.ki_sh;
  const int64_t st1 = is_q ? a.qi_st : a.ki_st;
  const int64_t o2 = (packed ? 0 : (int64_t)b * a.vi_sb) + (int64_t)hk * a.vi_sh;
  uint2 x1[kPasses], x2[kPasses], v1[kPasses], v2[kPasses], cw[kPasses], sw[kPasses];
  int64_t jp[kPasses];  // page index of the token's position
  int32_t phys[kPasses];
  bool valid[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int tu = tb + p * tpp + sub;
    // loads use the token clamped into the input rows; whenever the token is
    // valid below, tu <= tmax, so the clamp leaves it unchanged
    const int t = min(tu, tmax);
    const int64_t tr = packed ? max(min(r0 + t, a.num_rows - 1), (int64_t)0) : (int64_t)t;
    const int64_t pos = (int64_t)pos0 + t;
    const int64_t tp = pos < 0 ? 0 : (pos >= a.table_len ? a.table_len - 1 : pos);
    x1[p] = *reinterpret_cast<const uint2 *>(p1 + o1 + tr * st1 + e0);
    x2[p] = *reinterpret_cast<const uint2 *>(p1 + o1 + tr * st1 + half + e0);
    v1[p] = make_uint2(0u, 0u);
    v2[p] = make_uint2(0u, 0u);
    if (!is_q) {
      v1[p] = *reinterpret_cast<const uint2 *>(pv + o2 + tr * a.vi_st + e0);
      v2[p] = *reinterpret_cast<const uint2 *>(pv + o2 + tr * a.vi_st + half + e0);
    }
    cw[p] = *reinterpret_cast<const uint2 *>(tab + (tp << dsh) + e0);
    sw[p] = *reinterpret_cast<const uint2 *>(tab + (tp << dsh) + half + e0);
    const int64_t j = pos < 0 ? 0 : pos >> psh;
    jp[p] = j;
    phys[p] = (a.page_table != nullptr && !is_q)
                  ? a.page_table[(int64_t)b * a.max_pages + (j < a.max_pages ? j : a.max_pages - 1)]
                  : 0;
    bool ok = tu < a.num_new && pos >= 0 && pos < a.table_len;
    valid[p] = ok && (is_q ? (!packed || tu < nlen) : (tu < nlen && pos < a.capacity));
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int t = tb + p * tpp + sub;
    float xa[4], xb[4], c[4], sn[4], oa[4], ob[4];
    unpack4(x1[p], xa);
    unpack4(x2[p], xb);
    unpack4(cw[p], c);
    unpack4(sw[p], sn);
#pragma unroll
    for (int e = 0; e < 4; ++e) rotate_pair<BF16Tag>(xa[e], xb[e], c[e], sn[e], oa[e], ob[e]);
    if (is_q) {
      if (valid[p]) {
        uint16_t *q = static_cast<uint16_t *>(a.q_out) + (int64_t)b * a.qo_sb + (int64_t)row * a.qo_sh +
                      (int64_t)t * a.qo_st;
        *reinterpret_cast<uint2 *>(q + e0) = pack4(oa);
        *reinterpret_cast<uint2 *>(q + half + e0) = pack4(ob);
      }
      continue;
    }
    int64_t off = -1;  // slot offset, from the page entry loaded above
    if (valid[p]) {
      const int64_t j = jp[p];
      const int64_t pos = (int64_t)pos0 + t;
      const int64_t slot = pos - (j << psh);
      if (a.page_table == nullptr)
        off = (int64_t)b * a.c_seq + j * a.c_page + (int64_t)hk * a.c_head + (slot << dsh);
      else if (j < a.max_pages && phys[p] >= 0 && phys[p] < a.num_pages)
        off = (int64_t)phys[p] * a.c_page + (int64_t)hk * a.c_head + (slot << dsh);
    }
    if constexpr (!kFP8) {
      if (off >= 0) {
        uint16_t *kc = static_cast<uint16_t *>(a.k_cache);
        uint16_t *vc = static_cast<uint16_t *>(a.v_cache);
        *reinterpret_cast<uint2 *>(kc + off + e0) = pack4(oa);
        *reinterpret_cast<uint2 *>(kc + off + half + e0) = pack4(ob);
        *reinterpret_cast<uint2 *>(vc + off + e0) = v1[p];
        *reinterpret_cast<uint2 *>(vc + off + half + e0) = v2[p];
      }
    } else {
      // per-(token, head) symmetric scale over the token's lpt lanes
      float va[4], vb[4];
      unpack4(v1[p], va);
      unpack4(v2[p], vb);
      float km = 0.f, vm = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        km = absmax2(km, oa[e], ob[e]);
        vm = absmax2(vm, va[e], vb[e]);
      }
#pragma unroll
      for (int m = lpt >> 1; m > 0; m >>= 1) {
        km = __builtin_elementwise_maximum(km, __shfl_xor(km, m, 64));
        vm = __builtin_elementwise_maximum(vm, __shfl_xor(vm, m, 64));
      }
      const float ks = km / 448.0f;
      const float vs = vm / 448.0f;
      if (off >= 0) {
        const uint32_t ka = e4m3_row_codes4(oa, ks);
        const uint32_t kb = e4m3_row_codes4(ob, ks);
        const uint32_t wa = e4m3_row_codes4(va, vs);
        const uint32_t wb = e4m3_row_codes4(vb, vs);
        uint8_t *kc = static_cast<uint8_t *>(a.k_cache);
        uint8_t *vc = static_cast<uint8_t *>(a.v_cache);
        *reinterpret_cast<uint32_t *>(kc + off + e0) = ka;
        *reinterpret_cast<uint32_t *>(kc + off + half + e0) = kb;
        *reinterpret_cast<uint32_t *>(vc + off + e0) = wa;
        *reinterpret_cast<uint32_t *>(vc + off + half + e0) = wb;
        if (e0 == 0) {
          a.k_scale[fp8_scale_index(off >> dsh)] = ks;
          a.v_scale[fp8_scale_index(off >> dsh)] = vs;
        }
      }
    }
  }
}

// The vector kernel's access widths: 8-byte bf16 groups (4-byte fp8 codes).
bool vec_ok(const RopeAppendArgs &a) {
  const int D = a.head_dim;
  auto al = [](const void *p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; };
  const bool pow2 = D >= 16 && D <= 128 && (D & (D - 1)) == 0 && (a.page_size & (a.page_size - 1)) == 0;
  const int64_t st[] = {a.qi_sb, a.qi_sh, a.qi_st, a.ki_sb, a.ki_sh, a.ki_st, a.vi_sb, a.vi_sh, a.vi_st,
                        a.qo_sb, a.qo_sh, a.qo_st, a.c_seq, a.c_page, a.c_head};
  bool strides4 = true;
  for (int64_t x : st) strides4 = strides4 && x % 4 == 0;
  return pow2 && strides4 && al(a.q_in, 8) && al(a.k_in, 8) && al(a.v_in, 8) && al(a.q_out, 8) && al(a.table, 8) &&
         al(a.k_cache, 8) && al(a.v_cache, 8);
}

template <bool kFP8>
void launch_vec(const RopeAppendArgs &a, dim3 grid, hipStream_t stream) {
  switch (a.head_dim) {
    case 16: hipLaunchKernelGGL((rope_append_vec_kernel<kFP8, 4>), grid, dim3(64), 0, stream, a); break;
    case 32: hipLaunchKernelGGL((rope_append_vec_kernel<kFP8, 5>), grid, dim3(64), 0, stream, a); break;
    case 64: hipLaunchKernelGGL((rope_append_vec_kernel<kFP8, 6>), grid, dim3(64), 0, stream, a); break;
    default: hipLaunchKernelGGL((rope_append_vec_kernel<kFP8, 7>), grid, dim3(64), 0, stream, a); break;
  }
}

}  // namespace

hipError_t launch_rope_append(const RopeAppendArgs &a, CacheKind kind, hipStream_t stream) {
  if ((a.num_new > 1 || a.in_rows != nullptr) && a.part_splits <= 0) {
    if (kind != CacheKind::kF32 && vec_ok(a)) {
      const dim3 vgrid(a.hq + a.hkv, (a.num_new + kVecTok - 1) / kVecTok, a.batch);
      if (kind == CacheKind::kFP8)
        launch_vec<true>(a, vgrid, stream);
      else
        launch_vec<false>(a, vgrid, stream);
      return hipGetLastError();
    }
    const dim3 cgrid(a.hq + a.hkv, (a.num_new + kChunkTok - 1) / kChunkTok, a.batch);
    switch (kind) {
      case CacheKind::kBF16:
        hipLaunchKernelGGL((rope_append_chunk_kernel<BF16Tag, false>), cgrid, dim3(64), 0, stream, a);
        break;
      case CacheKind::kF32:
        hipLaunchKernelGGL((rope_append_chunk_kernel<float, false>), cgrid, dim3(64), 0, stream, a);
        break;
      case CacheKind::kFP8:
        hipLaunchKernelGGL((rope_append_chunk_kernel<BF16Tag, true>), cgrid, dim3(64), 0, stream, a);
        break;
    }
    return hipGetLastError();
  }
  const dim3 grid(a.hq + a.hkv, a.num_new > 0 ? a.num_new : 1, a.batch);
  const dim3 block(64);
  // split-K partial inputs: bf16 activations only (checked by the caller)
  const int part = a.part_splits <= 0 ? 0 : (a.part_splits <= 4 ? 1 : 2);
  switch (kind) {
    case CacheKind::kBF16:
      if (part == 1)
        hipLaunchKernelGGL((rope_append_kernel<BF16Tag, false, 1>), grid, block, 0, stream, a);
      else if (part == 2)
        hipLaunchKernelGGL((rope_append_kernel<BF16Tag, false, 2>), grid, block, 0, stream, a);
      else
        hipLaunchKernelGGL((rope_append_kernel<BF16Tag, false, 0>), grid, block, 0, stream, a);
      break;
    case CacheKind::kF32:
      hipLaunchKernelGGL((rope_append_kernel<float, false, 0>), grid, block, 0, stream, a);
      break;
    case CacheKind::kFP8:
      if (part == 1)
        hipLaunchKernelGGL((rope_append_kernel<BF16Tag, true, 1>), grid, block, 0, stream, a);
      else if (part == 2)
        hipLaunchKernelGGL((rope_append_kernel<BF16Tag, true, 2>), grid, block, 0, stream, a);
      else
        hipLaunchKernelGGL((rope_append_kernel<BF16Tag, true, 0>), grid, block, 0, stream, a);
      break;
  }
  return hipGetLastError();
}

}  // namespace tt
