// Internal launch interface between the C ABI layer (abi.hip) and the
// kernels (rope_append.hip, decode_attn.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace tt {

// Compute units of the current device, queried once per device (launch
// sizing reads it on every launch; the attribute query is not free).
inline int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < kMaxDevices) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev < kMaxDevices) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

enum class CacheKind { kBF16, kF32, kFP8 };

// fp8 caches keep their fp32 scales in groups of 16 rows (row = element
// offset of d = 0 / head_dim): rows 16g .. 16g + 15 have their K scales at
// 32g .. 32g + 15 of k_scale and their V scales at the same indices of
// v_scale, laid out so that one array of 2 x rows entries serves both with
// v_scale = k_scale + 16. A 16-token block's K and V scales then fill one
// 128-byte line, which the attention kernels read whole.
__host__ __device__ __forceinline__ int64_t fp8_scale_index(int64_t row) { return row + (row & ~(int64_t)15); }

struct RopeAppendArgs {
  const void *q_in;
  int64_t qi_sb, qi_sh, qi_st;
  const void *k_in;
  int64_t ki_sb, ki_sh, ki_st;
  const void *v_in;
  int64_t vi_sb, vi_sh, vi_st;
  void *q_out;
  int64_t qo_sb, qo_sh, qo_st;
  const void *table;
  int64_t table_len;
  const int32_t *positions;
  const int32_t *new_lens;
  int32_t *lens_out;
  const int32_t *page_table;
  int64_t max_pages, num_pages;
  void *k_cache;
  void *v_cache;
  float *k_scale;
  float *v_scale;
  int64_t c_seq, c_page, c_head;
  int64_t capacity;
  int batch, num_new, hq, hkv, head_dim, page_size;
  // q_in / k_in / v_in point into fp32 split-K partials (split stride part_stride
  // elements) when part_splits > 0: each input is bf16(sum of the splits, in order)
  int part_splits;
  int64_t part_stride;
  // packed prompt rows (in_rows != nullptr): token t of sequence b is input row
  // in_rows[b] + t (< num_rows) with row stride *_st and head stride *_sh (the
  // batch strides are unused); rows t >= new_lens[b] do not exist, so their q
  // rows are not written either
  const int32_t *in_rows;
  int64_t num_rows;
};

struct DecodeArgs {
  const void *q;
  int64_t q_sb, q_sh;
  const void *k_cache;
  const void *v_cache;
  const float *k_scale;
  const float *v_scale;
  int64_t c_seq, c_page, c_head;
  const int32_t *seq_lens;
  int max_len;
  const int32_t *page_table;
  int64_t max_pages, num_pages;
  void *out;
  int64_t o_sb, o_sh;
  float *ws_o;   // [B][H_kv][max_splits][G][D] unnormalised partial outputs
  float *ws_ml;  // [B][H_kv][max_splits][G][2] (running max in log2 units, sum)
                 // balanced partition (split_tokens == 0): [B * H_kv + kMaxStreamWaves][G][D] and [..][G][2]
  int32_t *ws_prefix;  // balanced partition: per-sequence tile prefix [B + 1], written by the split kernel
  // VALU kernel only: query row b reads the K/V of sequence seq_of_row[b]
  // (clamped into [0, num_seqs)) instead of sequence b (null: the identity)
  const int32_t *seq_of_row;
  int num_seqs;
  int stream_waves;    // balanced partition: waves of the split kernel's grid (set by the launcher)
  int batch, hq, hkv, group, split_tokens, max_splits;
  int page_shift;    // paged pools: log2(page_size); the contiguous store is addressed linearly
  float scale_log2;  // sm_scale * log2(e)
  int len_add;       // added to seq_lens[b] (1 when the kernel appends the step's token itself)
  // paired partition: the batch's sequence indices ordered by length (longest
  // first, ties by index), or null to rank them on the device
  const int32_t *order;
  // balanced partition: line positions charged to each (sequence, KV head) segment
  // before its tiles, so that a wave's share counts the fixed start-up cost of
  // every segment piece it holds, not only its tiles (set by the launcher)
  int seg_cost;
  // the cache's head_dim (row length) and 1 / head_dim; kernels built for a
  // wider tile (tile_head_dim) read rows of this length
  int head_dim;
  double inv_head_dim;
};

// Fused decode step: the split kernel also applies RoPE to this step's token
// (q, and k before it is written) and appends k / v to the cache, so that
// no separate RoPE + append launch precedes it. seq_lens holds the tokens
// cached before the step (len_add = 1).
struct DecodeAppend {
  const void *q_in, *k_in, *v_in;  // bf16 [B, H, D] views, or fp32 split-K partials
  int64_t qi_sb, qi_sh, ki_sb, ki_sh, vi_sb, vi_sh;
  int part_splits;  // 0: bf16 inputs; 1 .. kMaxApSplits: sum of the partials (stride part_stride) rounded to bf16
  int64_t part_stride;
  const void *table;  // RoPE table [table_len, D] bf16
  int64_t table_len;
  int32_t *lens_out;  // [B] lengths after the step, or null
  int64_t capacity;   // tokens per sequence the cache holds
  int64_t page_size;  // contiguous store: tokens per page (paged pools: 1 << page_shift)
};

constexpr int kMaxApSplits = 4;  // split-K partials the fused step sums per input

struct DecodeAppendArgs : DecodeArgs {
  DecodeAppend ap;
};

// Skinny GEMM of the decode step: partials P[K / kc][M][N] (fp32) of x[M, K] . W[N, K]^T.
struct SkinnyGemmArgs {
  const uint16_t *x;  // bf16 [M, K], row stride ldx
  int64_t ldx;
  const uint16_t *w;  // bf16 [N, K], row stride ldw
  int64_t ldw;
  float *part;
  int M, N, K;
  int packed;  // weights in fragment order [N/16][K/32][64][8] (ldw unused)
};

hipError_t launch_skinny_gemm(const SkinnyGemmArgs &a, int kc, hipStream_t stream);

// Gate|up projection + SwiGLU in one launch (weights: fragment-ordered, rows
// interleaved by 8 gate / 8 up); out [M, I] bf16, row stride ldo.
struct SwigluGemmArgs {
  const uint16_t *x;  // bf16 [M, K], row stride ldx
  int64_t ldx;
  const uint16_t *w;  // packed interleaved [2I/16][K/32][64][8]
  uint16_t *out;
  int64_t ldo;
  int M, I, K;
};
bool swiglu_gemm_supported(int64_t K, int64_t I);
hipError_t launch_swiglu_gemm(const SwigluGemmArgs &a, hipStream_t stream);
hipError_t launch_reduce_bf16(const float *P, int S, int64_t MN, uint16_t *y, hipStream_t stream);
hipError_t launch_add_rmsnorm(float *x, const float *P, int S, int M, int C, const float *w, float eps, uint16_t *y,
                              hipStream_t stream);
hipError_t launch_silu_mul(const float *P, int S, int M, int I, uint16_t *y, hipStream_t stream);
hipError_t launch_add_rmsnorm_rows(float *x, const uint16_t *a, int64_t lda, int M, int C, const float *w, float eps,
                                   uint16_t *y, hipStream_t stream);
hipError_t launch_silu_mul_rows(const uint16_t *g, int64_t ldg, const uint16_t *u, int64_t ldu, int64_t M, int I,
                                uint16_t *y, hipStream_t stream);

hipError_t launch_rope_append(const RopeAppendArgs &a, CacheKind kind, hipStream_t stream);
hipError_t launch_decode_attn(const DecodeArgs &a, CacheKind kind, int head_dim, hipStream_t stream);
hipError_t launch_decode_attn_append(const DecodeAppendArgs &a, CacheKind kind, int head_dim, hipStream_t stream);

// Prefill: T new tokens per sequence (their K/V already in the cache), causal
// GQA attention over each sequence's cached prefix. The cache fields, q / out
// pointers and scale come from DecodeArgs (out strides: o_sb = batch, o_sh = head).
struct PrefillArgs : DecodeArgs {
  int64_t q_st;                // q token stride
  int64_t o_st;                // out token stride
  const int32_t *positions;    // [B] tokens cached before the new ones
  const int32_t *new_lens;     // [B] new tokens per sequence (<= num_new), or null for all num_new
  int num_new;                 // T
  int qt;                      // query tokens per wave (16 / G)
  int nq;                      // query blocks per sequence: ceil(T / qt)
  int wg_per_pair;             // workgroups per (sequence, KV head): ceil(nq / 4)
  int vec_out;                 // out 8-byte aligned, strides multiples of 4: 4 head_dim entries per store
};

hipError_t launch_prefill_attn(const PrefillArgs &a, CacheKind kind, int head_dim, hipStream_t stream);

// Token sampling: one workgroup per row of logits [M, V] (bf16 or fp32).
struct SampleArgs {
  const void *logits;
  int64_t ld;           // row stride (elements)
  int M, V;             // V <= kMaxSampleVocabBF16 / kMaxSampleVocabF32
  int vec;              // rows 16-byte aligned: group loads are vector loads
  float temperature;
  int apply_temp;       // temperature != 1
  int top_k;            // <= 0: no top-k
  float top_p;
  int apply_top_p;      // 0 < top_p < 1
  uint64_t seed, offset;
  int64_t *tokens;      // [M]
  float *token_logprob; // [M] or null
  float *logprobs;      // [M, ld_lp] log-probabilities of the filtered logits, or null
  int64_t ld_lp;
  int vec_out;
  // Candidate path (top_k in [2, kCandSlots], no log-probability rows, V >
  // kCandChunk): workspace of M x cand_chunks CandRecords, or null.
  void *cand;
  int cand_chunks;
};

constexpr int kMaxSampleVocabBF16 = 65536;
constexpr int kMaxSampleVocabF32 = 32768;
constexpr int kCandChunk = 8192;  // logits per candidate workgroup
constexpr int kCandSlots = 64;    // candidates one chunk keeps (the largest top_k of the path)

// One chunk's candidates: its values >= its own k-th largest (all of those
// strictly above it, then ties in any order up to the slots; truncated when
// ties did not fit), the k-th largest's order key, and the values (after the
// temperature) with their row indices.
struct CandRecord {
  int count;
  int truncated;
  uint32_t kth_key;
  int pad;
  float val[kCandSlots];
  int32_t idx[kCandSlots];
};

hipError_t launch_sample(const SampleArgs &a, bool f32, hipStream_t stream);
// chunks of the candidate path for this call (0: the whole-row path runs alone);
// the candidate kernel puts rows in grid y, so more than kMaxCandRows rows take
// the whole-row path
constexpr int64_t kMaxCandRows = 65535;
int sample_cand_chunks(int64_t rows, int64_t vocab, int64_t top_k, bool logprobs_rows);

// Partition helpers shared by the ABI layer and the launchers.
int64_t auto_split_tokens(int64_t batch, int64_t hkv, int64_t max_len);
// split_tokens value of the per-segment partition: one workgroup per (sequence,
// KV head), merged in LDS, one launch, no workspace (MFMA kernels only).
constexpr int kSplitPerSegment = -1;
// Its grid, its dynamic LDS bytes, and the resident workgroups of one round on
// the current device (CUs x workgroups per CU at this tile width).
int64_t segment_grid(int64_t batch, int64_t hkv);
size_t segment_lds_bytes(int tile_d, bool fp8, bool fused, int64_t group);
int64_t segment_round(int tile_d);
// split_tokens value of the paired partition: the sequences ranked by length,
// workgroup (p, KV head) takes ranks p and B - 1 - p, its waves split the two
// segments' tiles, merged in LDS: one launch, no workspace, B <= kMaxPairedBatch.
constexpr int kSplitPaired = -2;
constexpr int64_t kMaxPairedBatch = 256;
// Its grid and dynamic LDS bytes (0: the GQA group does not fit in 64 KB).
int64_t paired_grid(int64_t batch, int64_t hkv);
size_t paired_lds_bytes(int tile_d, bool fp8, bool fused, int64_t group);
// Waves of the balanced stream kernel's grid on the current device (at most
// kMaxStreamWaves); the partial slots it writes are b * H_kv + hk + wave.
int64_t balanced_stream_waves(int head_dim, int64_t batch, int64_t hkv, int64_t max_len);
inline int64_t num_splits(int64_t max_len, int64_t split_tokens) {
  return max_len <= 0 ? 1 : (max_len + split_tokens - 1) / split_tokens;
}

// Tile width of the MFMA attention kernels for a bf16 / fp8 cache of this
// head_dim: the smallest of 32 (bf16 only), 64 and 128 that holds it, when a
// row is a whole number of 16-byte fragments (head_dim a multiple of 8 bf16 /
// 16 fp8 values) and head_dim <= 128; 0 otherwise (fp32 caches and other head
// dims take the VALU kernel).
inline int tile_head_dim(int64_t head_dim, CacheKind kind) {
  if (kind == CacheKind::kF32 || head_dim <= 0 || head_dim > 128) return 0;
  if (head_dim % (kind == CacheKind::kFP8 ? 16 : 8) != 0) return 0;
  if (kind == CacheKind::kBF16 && head_dim <= 32) return 32;
  return head_dim <= 64 ? 64 : 128;
}

// Width (floats) of the attention workspace's partial rows for any kernel and
// cache type: at least the tile width and head_dim.
inline int workspace_head_dim(int64_t head_dim, CacheKind = CacheKind::kBF16) { return head_dim <= 64 ? 64 : 128; }

constexpr int kWavesPerBlock = 4;
constexpr int kTileTokens = 32;  // tokens per wave iteration (two 16-row MFMA blocks)
constexpr int kMaxStreamBlocks = 1024;  // balanced partition: grid cap (>= 3 workgroups on each of 256 CUs)
constexpr int kMaxStreamWaves = kMaxStreamBlocks * kWavesPerBlock;
// balanced partition: tiles' worth of line positions charged to every (sequence,
// KV head) segment before its tiles (the start-up cost of a segment piece)
constexpr int kStreamSegCost = 2;

}  // namespace tt
