// extern "C" entry points of libtinytron_amd.so (declared in
// include/tinytron_amd.h): argument validation, status codes and launches.
// Nothing here allocates or synchronises; every launch goes on the caller's
// stream.
#include <algorithm>
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/tinytron_amd.h"
#include "tt_internal.h"

// Device scratch of tt_decode_attn_append_bf16_noalloc (the attention
// workspace: tile prefix, partial outputs, maxima and sums), one copy per
// GPU, held until the process ends. Its name is a host-side stand-in:
// kernels get its device address from scratch_address().
static __device__ __align__(256) unsigned char scratch[TT_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr size_t kScratchBytes = TT_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxScratchDevices = 64;
std::atomic<void *> g_scratch_addr[kMaxScratchDevices];
std::mutex g_scratch_mutex;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int from_hip(hipError_t err, const char *what);

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
int scratch_address(void **addr) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return from_hip(err, "hipGetDevice");
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(TT_ERR_UNSUPPORTED, "device %d is beyond the %d devices the scratch table covers", dev,
                kMaxScratchDevices);
  void *p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_addr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
      err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (err != hipSuccess || p == nullptr) return from_hip(err != hipSuccess ? err : hipErrorInvalidSymbol,
                                                             "hipGetSymbolAddress(scratch)");
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *addr = p;
  return TT_OK;
}

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return TT_OK;
}

int from_hip(hipError_t err, const char *what) {
  if (err == hipSuccess) return ok();
  g_last_error = std::string(what) + ": " + hipGetErrorString(err);
  return (int)err;
}

bool aligned(const void *p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

#define TT_CHECK(cond, code, ...) \
  do {                            \
    if (!(cond)) return fail(code, __VA_ARGS__); \
  } while (0)

int check_layout(const int32_t *page_table, int64_t max_pages, int64_t num_pages, const int64_t cache_strides[3],
                 int64_t page_size) {
  TT_CHECK(cache_strides != nullptr, TT_ERR_INVALID_ARGUMENT, "cache_strides is NULL");
  TT_CHECK(page_size > 0, TT_ERR_INVALID_ARGUMENT, "page_size must be positive, got %lld", (long long)page_size);
  TT_CHECK(cache_strides[1] >= 0 && cache_strides[2] >= 0 && cache_strides[0] >= 0, TT_ERR_INVALID_ARGUMENT,
           "cache strides must be non-negative");
  if (page_table != nullptr) {
    TT_CHECK(max_pages > 0 && num_pages > 0, TT_ERR_INVALID_ARGUMENT,
             "paged cache needs max_pages > 0 and num_pages > 0 (got %lld, %lld)", (long long)max_pages,
             (long long)num_pages);
  }
  return TT_OK;
}

// The contiguous store addresses token t of (b, h) at b * strides[0] +
// h * strides[2] + t * head_dim: the kernels read tokens below max_seq_len,
// so each (sequence, head) region must hold that many tokens. A stride whose
// dimension has more than one entry must be at least max_seq_len * head_dim
// (the reference's [B, H, pages, P, D] store has c_head = pages * P * D and
// c_seq = H * c_head).
// fp8 caches: one scale per row (strides multiples of head_dim), and every
// 16-token block of a (sequence, head) starting a 16-row scale group: page
// and head strides (pool) or sequence and head strides (contiguous store)
// multiples of 16 head_dim (tt::fp8_scale_index).
int check_fp8_strides(const int32_t *page_table, const int64_t cache_strides[3], int64_t head_dim) {
  TT_CHECK(cache_strides[0] % head_dim == 0 && cache_strides[1] % head_dim == 0 && cache_strides[2] % head_dim == 0,
           TT_ERR_INVALID_ARGUMENT, "fp8 cache strides must be multiples of head_dim (one scale per row)");
  const int64_t group = 16 * head_dim;
  const int64_t outer = page_table != nullptr ? cache_strides[1] : cache_strides[0];
  TT_CHECK(outer % group == 0 && cache_strides[2] % group == 0, TT_ERR_INVALID_ARGUMENT,
           "fp8 caches group their scales by 16 rows: the %s and head strides must be multiples of 16 * head_dim "
           "(a contiguous store's capacity a multiple of 16 tokens)", page_table != nullptr ? "page" : "sequence");
  return TT_OK;
}

int check_contiguous_room(int64_t max_seq_len, int64_t head_dim, const int64_t cache_strides[3], int64_t batch,
                          int64_t num_kv_heads) {
  const int64_t need = max_seq_len * head_dim;
  TT_CHECK(num_kv_heads <= 1 || cache_strides[2] >= need, TT_ERR_INVALID_ARGUMENT,
           "max_seq_len %lld does not fit the contiguous store: head stride %lld < %lld * head_dim",
           (long long)max_seq_len, (long long)cache_strides[2], (long long)max_seq_len);
  TT_CHECK(batch <= 1 || cache_strides[0] >= need, TT_ERR_INVALID_ARGUMENT,
           "max_seq_len %lld does not fit the contiguous store: sequence stride %lld < %lld * head_dim",
           (long long)max_seq_len, (long long)cache_strides[0], (long long)max_seq_len);
  return TT_OK;
}

int rope_append_common(tt::CacheKind kind, const void *q_in, const int64_t q_in_strides[3], const void *k_in,
                       const int64_t k_in_strides[3], const void *v_in, const int64_t v_in_strides[3], void *q_out,
                       const int64_t q_out_strides[3], const void *rope_table, int64_t rope_table_len,
                       const int32_t *positions, const int32_t *new_lens, int32_t *lens_out, const int32_t *page_table,
                       int64_t max_pages, int64_t num_pages, void *k_cache, void *v_cache, float *k_scale,
                       float *v_scale, const int64_t cache_strides[3], int64_t capacity, int64_t batch,
                       int64_t num_new, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                       int64_t page_size, tt_stream_t stream, int64_t part_splits = 0, int64_t part_stride = 0,
                       const int32_t *in_rows = nullptr, int64_t num_rows = 0) {
  TT_CHECK(q_in && k_in && v_in && q_out && rope_table && positions && k_cache && v_cache, TT_ERR_INVALID_ARGUMENT,
           "a required pointer is NULL");
  TT_CHECK(part_splits >= 0 && part_splits <= 4096 && (part_splits == 0 || part_stride > 0), TT_ERR_INVALID_ARGUMENT,
           "bad split-K partial description");
  TT_CHECK(part_splits == 0 || kind != tt::CacheKind::kF32, TT_ERR_UNSUPPORTED,
           "split-K partial inputs are for bf16 activations");
  TT_CHECK(q_in_strides && k_in_strides && v_in_strides && q_out_strides, TT_ERR_INVALID_ARGUMENT,
           "a stride array is NULL");
  TT_CHECK(batch >= 0 && num_new >= 0, TT_ERR_INVALID_ARGUMENT, "batch and num_new must be >= 0");
  TT_CHECK(num_q_heads > 0 && num_kv_heads > 0, TT_ERR_INVALID_ARGUMENT, "head counts must be positive");
  TT_CHECK(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 128, TT_ERR_UNSUPPORTED,
           "head_dim must be even and <= 128, got %lld", (long long)head_dim);
  TT_CHECK(rope_table_len >= 0 && capacity >= 0, TT_ERR_INVALID_ARGUMENT, "negative table length or capacity");
  TT_CHECK(batch <= 65535 && num_new <= 65535 && num_q_heads + num_kv_heads <= (1 << 30), TT_ERR_UNSUPPORTED,
           "grid too large");
  if (kind == tt::CacheKind::kFP8) {
    TT_CHECK(k_scale && v_scale, TT_ERR_INVALID_ARGUMENT, "fp8 cache needs k_scale and v_scale");
    TT_CHECK(cache_strides != nullptr, TT_ERR_INVALID_ARGUMENT, "a stride array is NULL");
    const int frc = check_fp8_strides(page_table, cache_strides, head_dim);
    if (frc != TT_OK) return frc;
  }
  TT_CHECK(lens_out == nullptr || ((const void *)lens_out != (const void *)positions &&
                                   (const void *)lens_out != (const void *)new_lens),
           TT_ERR_INVALID_ARGUMENT, "lens_out must not alias positions or new_lens");
  int rc = check_layout(page_table, max_pages, num_pages, cache_strides, page_size);
  if (rc != TT_OK) return rc;
  if (batch == 0) return ok();

  tt::RopeAppendArgs a{};
  a.q_in = q_in;
  a.qi_sb = q_in_strides[0];
  a.qi_sh = q_in_strides[1];
  a.qi_st = q_in_strides[2];
  a.k_in = k_in;
  a.ki_sb = k_in_strides[0];
  a.ki_sh = k_in_strides[1];
  a.ki_st = k_in_strides[2];
  a.v_in = v_in;
  a.vi_sb = v_in_strides[0];
  a.vi_sh = v_in_strides[1];
  a.vi_st = v_in_strides[2];
  a.q_out = q_out;
  a.qo_sb = q_out_strides[0];
  a.qo_sh = q_out_strides[1];
  a.qo_st = q_out_strides[2];
  a.table = rope_table;
  a.table_len = rope_table_len;
  a.positions = positions;
  a.new_lens = new_lens;
  a.lens_out = lens_out;
  a.page_table = page_table;
  a.max_pages = max_pages;
  a.num_pages = num_pages;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.c_seq = cache_strides[0];
  a.c_page = cache_strides[1];
  a.c_head = cache_strides[2];
  a.capacity = capacity;
  a.batch = (int)batch;
  a.num_new = (int)num_new;
  a.hq = (int)num_q_heads;
  a.hkv = (int)num_kv_heads;
  a.head_dim = (int)head_dim;
  a.page_size = (int)page_size;
  a.part_splits = (int)part_splits;
  a.part_stride = part_stride;
  a.in_rows = in_rows;
  a.num_rows = num_rows;
  (void)hipGetLastError();
  return from_hip(tt::launch_rope_append(a, kind, (hipStream_t)stream), "rope_append launch");
}

int64_t resolve_split(int64_t split_tokens, int64_t batch, int64_t hkv, int64_t max_len) {
  return split_tokens > 0 ? split_tokens : tt::auto_split_tokens(batch, hkv, max_len);
}

// Partial rows are tt::workspace_head_dim(head_dim) floats wide (every kernel's tile width fits).
size_t workspace_bytes(int64_t batch, int64_t hq, int64_t hkv, int64_t head_dim, int64_t max_len, int64_t split) {
  const int64_t g = hq / (hkv > 0 ? hkv : 1);
  const int64_t splits = tt::num_splits(max_len, split);
  const int64_t items = batch * hkv * splits * g;
  return (size_t)(items * tt::workspace_head_dim(head_dim) + items * 2) * sizeof(float);
}

// Balanced partition: the per-sequence tile prefix (padded to 16 bytes), then
// one partial slot per (segment + wave) index. Caller-provided workspaces are
// sized for the largest grid (kMaxStreamWaves waves, so that one size serves
// every device); the allocation-free entry point sizes its slots for the grid
// it launches.
int64_t balanced_slots(int64_t batch, int64_t hkv, int64_t waves) { return batch * hkv + waves; }
int64_t balanced_prefix_ints(int64_t batch) { return (batch + 1 + 3) & ~(int64_t)3; }

size_t balanced_workspace_bytes(int64_t batch, int64_t hq, int64_t hkv, int64_t head_dim,
                                int64_t waves = tt::kMaxStreamWaves) {
  const int64_t g = hq / (hkv > 0 ? hkv : 1);
  const int64_t rows = balanced_slots(batch, hkv, waves) * g;
  return (size_t)balanced_prefix_ints(batch) * sizeof(int32_t) +
         (size_t)(rows * tt::workspace_head_dim(head_dim) + rows * 2) * sizeof(float);
}

int decode_common(tt::CacheKind kind, const void *q, const int64_t q_strides[2], const void *k_cache,
                  const void *v_cache, const float *k_scale, const float *v_scale, const int64_t cache_strides[3],
                  const int32_t *seq_lens, int64_t max_seq_len, const int32_t *page_table, int64_t max_pages,
                  int64_t num_pages, void *out, const int64_t out_strides[2], int64_t batch, int64_t num_q_heads,
                  int64_t num_kv_heads, int64_t head_dim, int64_t page_size, float sm_scale, int64_t split_tokens,
                  void *workspace, size_t ws_bytes, tt_stream_t stream, const tt::DecodeAppend *ap = nullptr,
                  bool exact_slots = false, const int32_t *seq_of_row = nullptr, int64_t num_seqs = 0,
                  const int32_t *length_order = nullptr) {
  // ap != null: the fused step (q / k / v from ap, seq_lens = lengths before the step)
  // exact_slots: the balanced workspace holds slots for the launched grid only (allocation-free entry point)
  // seq_of_row != null: `batch` query rows, row b reading the cache of sequence seq_of_row[b] < num_seqs
  //   (the VALU kernel)
  TT_CHECK((ap || q) && k_cache && v_cache && seq_lens && out, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK((ap || q_strides) && out_strides, TT_ERR_INVALID_ARGUMENT, "a stride array is NULL");
  TT_CHECK(batch >= 0 && batch <= 65535, TT_ERR_INVALID_ARGUMENT, "batch must be in [0, 65535]");
  TT_CHECK(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0, TT_ERR_INVALID_ARGUMENT,
           "num_attention_heads must be divisible by num_key_value_heads");
  TT_CHECK(num_q_heads / num_kv_heads <= 16, TT_ERR_UNSUPPORTED, "GQA group size %lld > 16 is not supported",
           (long long)(num_q_heads / num_kv_heads));
  TT_CHECK(num_kv_heads <= 65535 && num_q_heads <= 65535, TT_ERR_UNSUPPORTED, "too many heads");
  TT_CHECK(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 128, TT_ERR_UNSUPPORTED,
           "head_dim must be even and <= 128, got %lld", (long long)head_dim);
  TT_CHECK(seq_of_row == nullptr || (ap == nullptr && num_seqs >= 1 && num_seqs <= INT32_MAX), TT_ERR_INVALID_ARGUMENT,
           "row attention needs 1 <= num_seqs <= INT32_MAX (got %lld)", (long long)num_seqs);
  // MFMA kernels on 32 / 64 / 128-wide tiles, or (0) the VALU kernel (which row attention always takes)
  const int tile = seq_of_row != nullptr ? 0 : tt::tile_head_dim(head_dim, kind);
  TT_CHECK(ap == nullptr || tile > 0, TT_ERR_UNSUPPORTED,
           "the fused decode step needs head_dim a multiple of 8 (bf16 cache) or 16 (fp8 cache), got %lld",
           (long long)head_dim);
  TT_CHECK(max_seq_len >= 0 && max_seq_len < (int64_t)1 << 30, TT_ERR_INVALID_ARGUMENT,
           "max_seq_len out of range");
  if (kind == tt::CacheKind::kFP8) {
    TT_CHECK(k_scale && v_scale, TT_ERR_INVALID_ARGUMENT, "fp8 cache needs k_scale and v_scale");
    const int frc = check_fp8_strides(page_table, cache_strides, head_dim);
    if (frc != TT_OK) return frc;
  }
  int rc = check_layout(page_table, max_pages, num_pages, cache_strides, page_size);
  if (rc != TT_OK) return rc;
  int page_shift = 0;
  if (page_table != nullptr) {
    while (page_shift < 30 && ((int64_t)1 << page_shift) < page_size) ++page_shift;
    TT_CHECK(page_size >= 16 && ((int64_t)1 << page_shift) == page_size, TT_ERR_UNSUPPORTED,
             "paged pools need a power-of-two page_size >= 16, got %lld", (long long)page_size);
    TT_CHECK(max_seq_len <= max_pages * page_size, TT_ERR_INVALID_ARGUMENT,
             "max_seq_len %lld exceeds the page table's %lld pages of %lld tokens", (long long)max_seq_len,
             (long long)max_pages, (long long)page_size);
  } else {
    TT_CHECK(cache_strides[1] == page_size * head_dim, TT_ERR_UNSUPPORTED,
             "the contiguous store needs dense pages (page stride %lld != page_size * head_dim)",
             (long long)cache_strides[1]);
    rc = check_contiguous_room(max_seq_len, head_dim, cache_strides, seq_of_row ? num_seqs : batch, num_kv_heads);
    if (rc != TT_OK) return rc;
  }
  if (tile > 0) {
    TT_CHECK(batch <= 4096, TT_ERR_UNSUPPORTED, "batch %lld > 4096 is not supported (per-sequence split table in LDS)",
             (long long)batch);
    TT_CHECK((ap || aligned(q, 16)) && aligned(k_cache, 16) && aligned(v_cache, 16), TT_ERR_INVALID_ARGUMENT,
             "q and cache pointers must be 16-byte aligned");
    TT_CHECK(ap || (q_strides[0] % 8 == 0 && q_strides[1] % 8 == 0), TT_ERR_INVALID_ARGUMENT,
             "q strides must be multiples of 8 elements");
    TT_CHECK(cache_strides[0] % 8 == 0 && cache_strides[1] % 8 == 0 && cache_strides[2] % 8 == 0,
             TT_ERR_INVALID_ARGUMENT, "cache strides must be multiples of 8 elements");
  } else {
    const size_t qa = kind == tt::CacheKind::kF32 ? 4 : 2;
    const size_t ca = kind == tt::CacheKind::kF32 ? 4 : (kind == tt::CacheKind::kBF16 ? 2 : 1);
    TT_CHECK(aligned(q, qa) && aligned(k_cache, ca) && aligned(v_cache, ca) && aligned(out, qa),
             TT_ERR_INVALID_ARGUMENT, "q, cache and out pointers must be aligned to their element size");
  }
  // On the MFMA path split_tokens 0 is the balanced partition (equal tiles per
  // wave), kSplitPerSegment one workgroup per segment and kSplitPaired one per
  // pair of length ranks; the VALU kernel takes all three as 0 (its automatic
  // fixed split). Otherwise fixed splits.
  TT_CHECK(split_tokens >= tt::kSplitPaired, TT_ERR_INVALID_ARGUMENT,
           "split_tokens must be 0 (auto), %d (per segment), %d (paired), 128, 256, 512 or 1024, got %lld",
           tt::kSplitPerSegment, tt::kSplitPaired, (long long)split_tokens);
  if (split_tokens < 0 && tile == 0) split_tokens = 0;
  const bool segment = split_tokens < 0;  // the one-launch partitions, no workspace
  const bool balanced = split_tokens == 0 && tile > 0;
  int64_t split = 0, splits = 0;
  size_t need = 0;
  // partial slots beyond the segments: one per wave of the largest grid, or of the launched one
  const int64_t ws_waves =
      exact_slots ? tt::balanced_stream_waves(tile, batch, num_kv_heads, max_seq_len) : tt::kMaxStreamWaves;
  if (segment) {
    TT_CHECK(batch * num_kv_heads <= INT32_MAX, TT_ERR_UNSUPPORTED, "batch * num_kv_heads is too large");
    if (split_tokens == tt::kSplitPaired) {
      TT_CHECK(batch <= tt::kMaxPairedBatch, TT_ERR_UNSUPPORTED, "the paired partition takes at most %lld sequences, got %lld",
               (long long)tt::kMaxPairedBatch, (long long)batch);
      TT_CHECK(tt::paired_lds_bytes(tile, kind == tt::CacheKind::kFP8, ap != nullptr, num_q_heads / num_kv_heads) > 0,
               TT_ERR_UNSUPPORTED, "the paired partition's LDS does not fit this GQA group (%lld) and head_dim",
               (long long)(num_q_heads / num_kv_heads));
    }
    split = split_tokens;  // no workspace
  } else if (balanced) {
    // the per-sequence line prefix (int32) counts each sequence's tiles plus its segment start-up charge
    TT_CHECK(batch * ((max_seq_len + tt::kTileTokens - 1) / tt::kTileTokens + tt::kStreamSegCost) < ((int64_t)1 << 31),
             TT_ERR_UNSUPPORTED, "batch * max_seq_len is too large for the balanced partition");
    need = balanced_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, ws_waves);
  } else {
    split = resolve_split(split_tokens, batch, num_kv_heads, max_seq_len);
    TT_CHECK(split == 128 || split == 256 || split == 512 || split == 1024, TT_ERR_INVALID_ARGUMENT,
             "split_tokens must be 0 (auto), 128, 256, 512 or 1024, got %lld", (long long)split_tokens);
    splits = tt::num_splits(max_seq_len, split);
    TT_CHECK(splits <= 65535, TT_ERR_UNSUPPORTED, "too many splits (%lld)", (long long)splits);
    need = workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, max_seq_len, split);
  }
  TT_CHECK(need == 0 || (workspace != nullptr && ws_bytes >= need), TT_ERR_WORKSPACE_TOO_SMALL,
           "%s of %zu bytes is smaller than the %zu bytes needed",
           exact_slots ? "the allocation-free entry point's scratch" : "workspace", ws_bytes, need);
  TT_CHECK(aligned(workspace, 16), TT_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  if (batch == 0) return ok();

  tt::DecodeArgs a{};
  a.q = q;
  a.q_sb = ap ? 0 : q_strides[0];
  a.q_sh = ap ? 0 : q_strides[1];
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.c_seq = cache_strides[0];
  a.c_page = cache_strides[1];
  a.c_head = cache_strides[2];
  a.seq_lens = seq_lens;
  a.max_len = (int)max_seq_len;
  a.page_table = page_table;
  a.max_pages = max_pages;
  a.num_pages = num_pages;
  a.out = out;
  a.o_sb = out_strides[0];
  a.o_sh = out_strides[1];
  const int64_t g = num_q_heads / num_kv_heads;
  if (!segment) {
    const int64_t rows = g * (balanced ? balanced_slots(batch, num_kv_heads, ws_waves) : batch * num_kv_heads * splits);
    a.ws_prefix = balanced ? static_cast<int32_t *>(workspace) : nullptr;
    a.ws_o = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                       (balanced ? balanced_prefix_ints(batch) * sizeof(int32_t) : 0));
    a.ws_ml = a.ws_o + rows * tt::workspace_head_dim(head_dim);
  }
  a.head_dim = (int)head_dim;
  a.inv_head_dim = 1.0 / (double)head_dim;
  a.seq_of_row = seq_of_row;
  a.num_seqs = (int)num_seqs;
  a.batch = (int)batch;
  a.hq = (int)num_q_heads;
  a.hkv = (int)num_kv_heads;
  a.group = (int)g;
  a.page_shift = page_shift;
  a.split_tokens = (int)split;
  a.max_splits = (int)splits;
  a.order = split == tt::kSplitPaired ? length_order : nullptr;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  (void)hipGetLastError();
  if (ap != nullptr) {
    tt::DecodeAppendArgs f{};
    static_cast<tt::DecodeArgs &>(f) = a;
    f.len_add = 1;
    f.ap = *ap;
    return from_hip(tt::launch_decode_attn_append(f, kind, (int)head_dim, (hipStream_t)stream),
                    "fused decode attention launch");
  }
  return from_hip(tt::launch_decode_attn(a, kind, (int)head_dim, (hipStream_t)stream), "decode attention launch");
}

// The fused decode step: RoPE + append of this step's token inside the
// attention launch (q_in / k_in / v_in: bf16 [B, H, D] views, or with
// splits > 0 fp32 split-K partials).
int decode_append_common(tt::CacheKind kind, const void *q_in, const int64_t q_in_strides[2], const void *k_in,
                         const int64_t k_in_strides[2], const void *v_in, const int64_t v_in_strides[2],
                         int64_t splits, int64_t split_stride, const void *rope_table, int64_t rope_table_len,
                         const int32_t *positions, int32_t *lens_out, int64_t max_seq_len, const int32_t *page_table,
                         int64_t max_pages, int64_t num_pages, void *k_cache, void *v_cache, float *k_scale,
                         float *v_scale, const int64_t cache_strides[3], int64_t capacity, void *out,
                         const int64_t out_strides[2], int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                         int64_t head_dim, int64_t page_size, float sm_scale, int64_t split_tokens,
                         const int32_t *length_order, void *workspace, size_t ws_bytes, tt_stream_t stream,
                         bool exact_slots = false) {
  TT_CHECK(q_in && k_in && v_in && rope_table && positions, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(split_tokens == 0 || split_tokens == tt::kSplitPerSegment || split_tokens == tt::kSplitPaired,
           TT_ERR_INVALID_ARGUMENT,
           "the fused decode step takes split_tokens 0 (balanced), %d (per segment) or %d (paired), got %lld",
           tt::kSplitPerSegment, tt::kSplitPaired, (long long)split_tokens);
  TT_CHECK(q_in_strides && k_in_strides && v_in_strides, TT_ERR_INVALID_ARGUMENT, "a stride array is NULL");
  TT_CHECK(splits >= 0 && (splits == 0 || split_stride > 0), TT_ERR_INVALID_ARGUMENT, "bad split-K partial layout");
  TT_CHECK(splits <= tt::kMaxApSplits, TT_ERR_UNSUPPORTED, "the fused step sums at most %d split-K partials, got %lld",
           tt::kMaxApSplits, (long long)splits);
  TT_CHECK(rope_table_len >= 1 && capacity >= 1, TT_ERR_INVALID_ARGUMENT, "empty RoPE table or cache");
  TT_CHECK(max_seq_len >= 1 && max_seq_len <= capacity, TT_ERR_INVALID_ARGUMENT,
           "max_seq_len must bound the lengths after the step (1 .. capacity)");
  TT_CHECK(lens_out == nullptr || (const void *)lens_out != (const void *)positions, TT_ERR_INVALID_ARGUMENT,
           "lens_out must not alias positions");
  tt::DecodeAppend ap{};
  ap.q_in = q_in;
  ap.k_in = k_in;
  ap.v_in = v_in;
  ap.qi_sb = q_in_strides[0];
  ap.qi_sh = q_in_strides[1];
  ap.ki_sb = k_in_strides[0];
  ap.ki_sh = k_in_strides[1];
  ap.vi_sb = v_in_strides[0];
  ap.vi_sh = v_in_strides[1];
  ap.part_splits = (int)splits;
  ap.part_stride = split_stride;
  ap.table = rope_table;
  ap.table_len = rope_table_len;
  ap.lens_out = lens_out;
  ap.capacity = capacity;
  ap.page_size = page_size;
  return decode_common(kind, nullptr, nullptr, k_cache, v_cache, k_scale, v_scale, cache_strides, positions,
                       max_seq_len, page_table, max_pages, num_pages, out, out_strides, batch, num_q_heads,
                       num_kv_heads, head_dim, page_size, sm_scale, split_tokens, workspace, ws_bytes, stream, &ap,
                       exact_slots, nullptr, 0, length_order);
}

int linear_common(const void *x, int64_t ldx, const void *weight, int64_t ldw, int packed, float *partials,
                  int64_t m, int64_t n, int64_t k, int64_t k_chunk, tt_stream_t stream) {
  TT_CHECK(x && weight && partials, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(m >= 0 && m <= 65535 * 64 && n > 0 && k > 0, TT_ERR_INVALID_ARGUMENT, "bad GEMM shape");
  TT_CHECK(k_chunk == 256 || k_chunk == 512 || k_chunk == 1024, TT_ERR_INVALID_ARGUMENT,
           "k_chunk must be 256, 512 or 1024, got %lld", (long long)k_chunk);
  TT_CHECK(n % 64 == 0 && k % k_chunk == 0, TT_ERR_UNSUPPORTED,
           "N must be a multiple of 64 and K of k_chunk (N %lld, K %lld, k_chunk %lld)", (long long)n, (long long)k,
           (long long)k_chunk);
  TT_CHECK(n < ((int64_t)1 << 31) && k < ((int64_t)1 << 31), TT_ERR_UNSUPPORTED, "GEMM dimension too large");
  TT_CHECK(ldx >= k && ldw >= k && ldx % 8 == 0 && ldw % 8 == 0, TT_ERR_INVALID_ARGUMENT,
           "row strides must be >= K and multiples of 8 elements");
  TT_CHECK(aligned(x, 16) && aligned(weight, 16) && aligned(partials, 16), TT_ERR_INVALID_ARGUMENT,
           "x, weight and partials must be 16-byte aligned");
  if (m == 0) return ok();
  tt::SkinnyGemmArgs a{};
  a.x = static_cast<const uint16_t *>(x);
  a.ldx = ldx;
  a.w = static_cast<const uint16_t *>(weight);
  a.ldw = ldw;
  a.part = partials;
  a.M = (int)m;
  a.N = (int)n;
  a.K = (int)k;
  a.packed = packed;
  (void)hipGetLastError();
  return from_hip(tt::launch_skinny_gemm(a, (int)k_chunk, (hipStream_t)stream), "linear launch");
}
int prefill_common(tt::CacheKind kind, const void *q, const int64_t q_strides[3], const void *k_cache,
                   const void *v_cache, const float *k_scale, const float *v_scale, const int64_t cache_strides[3],
                   const int32_t *positions, const int32_t *new_lens, int64_t max_seq_len, const int32_t *page_table,
                   int64_t max_pages, int64_t num_pages, void *out, const int64_t out_strides[3], int64_t batch,
                   int64_t num_new, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                   float sm_scale, tt_stream_t stream) {
  TT_CHECK(q && k_cache && v_cache && positions && out, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(q_strides && out_strides, TT_ERR_INVALID_ARGUMENT, "a stride array is NULL");
  TT_CHECK(batch >= 0 && num_new >= 0, TT_ERR_INVALID_ARGUMENT, "batch and num_new must be >= 0");
  TT_CHECK(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0, TT_ERR_INVALID_ARGUMENT,
           "num_attention_heads must be divisible by num_key_value_heads");
  const int64_t g = num_q_heads / num_kv_heads;
  TT_CHECK(g <= 16, TT_ERR_UNSUPPORTED, "GQA group size %lld > 16 is not supported", (long long)g);
  TT_CHECK(tt::tile_head_dim(head_dim, kind) > 0, TT_ERR_UNSUPPORTED,
           "prefill attention needs head_dim <= 128 and a multiple of 8 (bf16 cache) or 16 (fp8 cache), got %lld",
           (long long)head_dim);
  TT_CHECK(max_seq_len >= 0 && max_seq_len < ((int64_t)1 << 30), TT_ERR_INVALID_ARGUMENT, "max_seq_len out of range");
  TT_CHECK(batch * num_kv_heads < ((int64_t)1 << 26) && num_new < ((int64_t)1 << 24), TT_ERR_UNSUPPORTED,
           "grid too large");
  if (kind == tt::CacheKind::kFP8) {
    TT_CHECK(k_scale && v_scale, TT_ERR_INVALID_ARGUMENT, "fp8 cache needs k_scale and v_scale");
    const int frc = check_fp8_strides(page_table, cache_strides, head_dim);
    if (frc != TT_OK) return frc;
  }
  int rc = check_layout(page_table, max_pages, num_pages, cache_strides, page_size);
  if (rc != TT_OK) return rc;
  int page_shift = 0;
  if (page_table != nullptr) {
    while (page_shift < 30 && ((int64_t)1 << page_shift) < page_size) ++page_shift;
    TT_CHECK(page_size >= 16 && ((int64_t)1 << page_shift) == page_size, TT_ERR_UNSUPPORTED,
             "paged pools need a power-of-two page_size >= 16, got %lld", (long long)page_size);
    TT_CHECK(max_seq_len <= max_pages * page_size, TT_ERR_INVALID_ARGUMENT,
             "max_seq_len %lld exceeds the page table's %lld pages of %lld tokens", (long long)max_seq_len,
             (long long)max_pages, (long long)page_size);
  } else {
    TT_CHECK(cache_strides[1] == page_size * head_dim, TT_ERR_UNSUPPORTED,
             "the contiguous store needs dense pages (page stride %lld != page_size * head_dim)",
             (long long)cache_strides[1]);
    rc = check_contiguous_room(max_seq_len, head_dim, cache_strides, batch, num_kv_heads);
    if (rc != TT_OK) return rc;
  }
  TT_CHECK(aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16), TT_ERR_INVALID_ARGUMENT,
           "q and cache pointers must be 16-byte aligned");
  TT_CHECK(q_strides[0] % 8 == 0 && q_strides[1] % 8 == 0 && q_strides[2] % 8 == 0, TT_ERR_INVALID_ARGUMENT,
           "q strides must be multiples of 8 elements");
  TT_CHECK(cache_strides[0] % 8 == 0 && cache_strides[1] % 8 == 0 && cache_strides[2] % 8 == 0,
           TT_ERR_INVALID_ARGUMENT, "cache strides must be multiples of 8 elements");
  if (batch == 0 || num_new == 0) return ok();

  tt::PrefillArgs a{};
  a.q = q;
  a.q_sb = q_strides[0];
  a.q_sh = q_strides[1];
  a.q_st = q_strides[2];
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.c_seq = cache_strides[0];
  a.c_page = cache_strides[1];
  a.c_head = cache_strides[2];
  a.max_len = (int)max_seq_len;
  a.page_table = page_table;
  a.max_pages = max_pages;
  a.num_pages = num_pages;
  a.out = out;
  a.o_sb = out_strides[0];
  a.o_st = out_strides[1];
  a.o_sh = out_strides[2];
  a.vec_out = aligned(out, 8) && out_strides[0] % 4 == 0 && out_strides[1] % 4 == 0 && out_strides[2] % 4 == 0;
  a.batch = (int)batch;
  a.hq = (int)num_q_heads;
  a.hkv = (int)num_kv_heads;
  a.group = (int)g;
  a.page_shift = page_shift;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.head_dim = (int)head_dim;
  a.inv_head_dim = 1.0 / (double)head_dim;
  a.positions = positions;
  a.new_lens = new_lens;
  a.num_new = (int)num_new;
  a.qt = (int)(16 / g);
  a.nq = (int)((num_new + a.qt - 1) / a.qt);
  a.wg_per_pair = (a.nq + tt::kWavesPerBlock - 1) / tt::kWavesPerBlock;
  (void)hipGetLastError();
  return from_hip(tt::launch_prefill_attn(a, kind, (int)head_dim, (hipStream_t)stream), "prefill attention launch");
}

int sample_common(bool f32, const void *logits, int64_t ld, int64_t m, int64_t vocab, float temperature,
                  int64_t top_k, float top_p, uint64_t seed, uint64_t offset, int64_t *tokens, float *token_logprob,
                  float *logprobs, int64_t ld_logprobs, void *workspace, size_t workspace_bytes,
                  tt_stream_t stream) {
  TT_CHECK(temperature > 0.f, TT_ERR_INVALID_ARGUMENT, "temperature must be > 0");
  TT_CHECK(m >= 0 && m <= INT32_MAX, TT_ERR_INVALID_ARGUMENT, "rows must be in [0, 2^31)");
  if (m == 0) return ok();
  TT_CHECK(logits && tokens, TT_ERR_INVALID_ARGUMENT, "logits and tokens are required");
  const int64_t vmax = f32 ? tt::kMaxSampleVocabF32 : tt::kMaxSampleVocabBF16;
  TT_CHECK(vocab >= 1 && vocab <= vmax, TT_ERR_UNSUPPORTED, "vocab size %lld outside [1, %lld]", (long long)vocab,
           (long long)vmax);
  TT_CHECK(ld >= vocab, TT_ERR_INVALID_ARGUMENT, "logits row stride %lld < vocab %lld", (long long)ld,
           (long long)vocab);
  TT_CHECK(logprobs == nullptr || ld_logprobs >= vocab, TT_ERR_INVALID_ARGUMENT,
           "logprobs row stride %lld < vocab %lld", (long long)ld_logprobs, (long long)vocab);
  const int64_t esize = f32 ? 4 : 2;
  tt::SampleArgs a{};
  a.logits = logits;
  a.ld = ld;
  a.M = (int)m;
  a.V = (int)vocab;
  a.vec = aligned(logits, 16) && (ld * esize) % 16 == 0;
  a.temperature = temperature;
  a.apply_temp = temperature != 1.0f;
  a.top_k = top_k > 0 ? (int)(top_k < vocab ? top_k : vocab) : 0;
  a.top_p = top_p;
  a.apply_top_p = top_p > 0.f && top_p < 1.0f;
  a.seed = seed;
  a.offset = offset;
  a.tokens = tokens;
  a.token_logprob = token_logprob;
  a.logprobs = logprobs;
  a.ld_lp = ld_logprobs;
  a.vec_out = logprobs != nullptr && aligned(logprobs, 16) && ld_logprobs % 4 == 0;
  a.cand_chunks = tt::sample_cand_chunks(m, vocab, a.top_k, logprobs != nullptr);
  a.cand = nullptr;
  if (workspace != nullptr && a.cand_chunks > 0) {
    const size_t need = (size_t)m * a.cand_chunks * sizeof(tt::CandRecord);
    TT_CHECK(workspace_bytes >= need, TT_ERR_WORKSPACE_TOO_SMALL,
             "sampler workspace of %zu bytes is smaller than the %zu this call needs", workspace_bytes, need);
    TT_CHECK(aligned(workspace, 16), TT_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    a.cand = workspace;
  }
  (void)hipGetLastError();
  return from_hip(tt::launch_sample(a, f32, (hipStream_t)stream), "sampler launch");
}

}  // namespace

extern "C" {

int tt_abi_version(void) { return TT_ABI_VERSION; }

const char *tt_last_error_string(void) { return g_last_error.c_str(); }

int tt_rope_append_bf16(const void *q_in, const int64_t q_in_strides[3], const void *k_in,
                        const int64_t k_in_strides[3], const void *v_in, const int64_t v_in_strides[3], void *q_out,
                        const int64_t q_out_strides[3], const void *rope_table, int64_t rope_table_len,
                        const int32_t *positions, const int32_t *new_lens, int32_t *lens_out, const int32_t *page_table,
                        int64_t max_pages, int64_t num_pages, void *k_cache, void *v_cache,
                        const int64_t cache_strides[3], int64_t capacity, int64_t batch, int64_t num_new,
                        int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                        tt_stream_t stream) {
  return rope_append_common(tt::CacheKind::kBF16, q_in, q_in_strides, k_in, k_in_strides, v_in, v_in_strides, q_out,
                            q_out_strides, rope_table, rope_table_len, positions, new_lens, lens_out, page_table, max_pages,
                            num_pages, k_cache, v_cache, nullptr, nullptr, cache_strides, capacity, batch, num_new,
                            num_q_heads, num_kv_heads, head_dim, page_size, stream);
}

int tt_rope_append_f32(const void *q_in, const int64_t q_in_strides[3], const void *k_in,
                       const int64_t k_in_strides[3], const void *v_in, const int64_t v_in_strides[3], void *q_out,
                       const int64_t q_out_strides[3], const void *rope_table, int64_t rope_table_len,
                       const int32_t *positions, const int32_t *new_lens, int32_t *lens_out, const int32_t *page_table,
                       int64_t max_pages, int64_t num_pages, void *k_cache, void *v_cache,
                       const int64_t cache_strides[3], int64_t capacity, int64_t batch, int64_t num_new,
                       int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                       tt_stream_t stream) {
  return rope_append_common(tt::CacheKind::kF32, q_in, q_in_strides, k_in, k_in_strides, v_in, v_in_strides, q_out,
                            q_out_strides, rope_table, rope_table_len, positions, new_lens, lens_out, page_table, max_pages,
                            num_pages, k_cache, v_cache, nullptr, nullptr, cache_strides, capacity, batch, num_new,
                            num_q_heads, num_kv_heads, head_dim, page_size, stream);
}

int tt_rope_append_fp8(const void *q_in, const int64_t q_in_strides[3], const void *k_in,
                       const int64_t k_in_strides[3], const void *v_in, const int64_t v_in_strides[3], void *q_out,
                       const int64_t q_out_strides[3], const void *rope_table, int64_t rope_table_len,
                       const int32_t *positions, const int32_t *new_lens, int32_t *lens_out, const int32_t *page_table,
                       int64_t max_pages, int64_t num_pages, void *k_cache, void *v_cache, float *k_scale,
                       float *v_scale, const int64_t cache_strides[3], int64_t capacity, int64_t batch,
                       int64_t num_new, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                       int64_t page_size, tt_stream_t stream) {
  return rope_append_common(tt::CacheKind::kFP8, q_in, q_in_strides, k_in, k_in_strides, v_in, v_in_strides, q_out,
                            q_out_strides, rope_table, rope_table_len, positions, new_lens, lens_out, page_table, max_pages,
                            num_pages, k_cache, v_cache, k_scale, v_scale, cache_strides, capacity, batch, num_new,
                            num_q_heads, num_kv_heads, head_dim, page_size, stream);
}

int tt_rope_append_rows_bf16(const void *q_in, const int64_t q_in_strides[2], const void *k_in,
                             const int64_t k_in_strides[2], const void *v_in, const int64_t v_in_strides[2],
                             const int32_t *row_offsets, int64_t num_rows, void *q_out, const int64_t q_out_strides[3],
                             const void *rope_table, int64_t rope_table_len, const int32_t *positions,
                             const int32_t *new_lens, int32_t *lens_out, const int32_t *page_table, int64_t max_pages,
                             int64_t num_pages, void *k_cache, void *v_cache, float *k_scale, float *v_scale,
                             const int64_t cache_strides[3], int64_t capacity, int64_t batch, int64_t num_new,
                             int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                             int fp8_cache, tt_stream_t stream) {
  TT_CHECK(row_offsets && new_lens, TT_ERR_INVALID_ARGUMENT, "packed rows need row_offsets and new_lens");
  TT_CHECK(num_rows >= 1 && num_rows <= INT32_MAX, TT_ERR_INVALID_ARGUMENT, "num_rows must be in [1, 2^31)");
  TT_CHECK(q_in_strides && k_in_strides && v_in_strides, TT_ERR_INVALID_ARGUMENT, "a stride array is NULL");
  const int64_t qs[3] = {0, q_in_strides[1], q_in_strides[0]};
  const int64_t ks[3] = {0, k_in_strides[1], k_in_strides[0]};
  const int64_t vs[3] = {0, v_in_strides[1], v_in_strides[0]};
  return rope_append_common(fp8_cache ? tt::CacheKind::kFP8 : tt::CacheKind::kBF16, q_in, qs, k_in, ks, v_in, vs,
                            q_out, q_out_strides, rope_table, rope_table_len, positions, new_lens, lens_out, page_table,
                            max_pages, num_pages, k_cache, v_cache, k_scale, v_scale, cache_strides, capacity, batch,
                            num_new, num_q_heads, num_kv_heads, head_dim, page_size, stream, 0, 0, row_offsets,
                            num_rows);
}

int tt_rope_append_partials_bf16(const float *q_in, const int64_t q_in_strides[3], const float *k_in,
                                 const int64_t k_in_strides[3], const float *v_in, const int64_t v_in_strides[3],
                                 int64_t splits, int64_t split_stride, void *q_out, const int64_t q_out_strides[3],
                                 const void *rope_table, int64_t rope_table_len, const int32_t *positions,
                                 const int32_t *new_lens, int32_t *lens_out, const int32_t *page_table,
                                 int64_t max_pages, int64_t num_pages, void *k_cache, void *v_cache,
                                 const int64_t cache_strides[3], int64_t capacity, int64_t batch, int64_t num_new,
                                 int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                 tt_stream_t stream) {
  TT_CHECK(splits >= 1, TT_ERR_INVALID_ARGUMENT, "splits must be >= 1");
  return rope_append_common(tt::CacheKind::kBF16, q_in, q_in_strides, k_in, k_in_strides, v_in, v_in_strides, q_out,
                            q_out_strides, rope_table, rope_table_len, positions, new_lens, lens_out, page_table,
                            max_pages, num_pages, k_cache, v_cache, nullptr, nullptr, cache_strides, capacity, batch,
                            num_new, num_q_heads, num_kv_heads, head_dim, page_size, stream, splits, split_stride);
}

int tt_rope_append_partials_fp8(const float *q_in, const int64_t q_in_strides[3], const float *k_in,
                                const int64_t k_in_strides[3], const float *v_in, const int64_t v_in_strides[3],
                                int64_t splits, int64_t split_stride, void *q_out, const int64_t q_out_strides[3],
                                const void *rope_table, int64_t rope_table_len, const int32_t *positions,
                                const int32_t *new_lens, int32_t *lens_out, const int32_t *page_table,
                                int64_t max_pages, int64_t num_pages, void *k_cache, void *v_cache, float *k_scale,
                                float *v_scale, const int64_t cache_strides[3], int64_t capacity, int64_t batch,
                                int64_t num_new, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                int64_t page_size, tt_stream_t stream) {
  TT_CHECK(splits >= 1, TT_ERR_INVALID_ARGUMENT, "splits must be >= 1");
  return rope_append_common(tt::CacheKind::kFP8, q_in, q_in_strides, k_in, k_in_strides, v_in, v_in_strides, q_out,
                            q_out_strides, rope_table, rope_table_len, positions, new_lens, lens_out, page_table,
                            max_pages, num_pages, k_cache, v_cache, k_scale, v_scale, cache_strides, capacity, batch,
                            num_new, num_q_heads, num_kv_heads, head_dim, page_size, stream, splits, split_stride);
}

int tt_prefill_attn_bf16(const void *q, const int64_t q_strides[3], const void *k_cache, const void *v_cache,
                         const int64_t cache_strides[3], const int32_t *positions, const int32_t *new_lens,
                         int64_t max_seq_len, const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                         void *out, const int64_t out_strides[3], int64_t batch, int64_t num_new,
                         int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                         float sm_scale, tt_stream_t stream) {
  return prefill_common(tt::CacheKind::kBF16, q, q_strides, k_cache, v_cache, nullptr, nullptr, cache_strides,
                        positions, new_lens, max_seq_len, page_table, max_pages, num_pages, out, out_strides, batch,
                        num_new, num_q_heads, num_kv_heads, head_dim, page_size, sm_scale, stream);
}

int tt_prefill_attn_fp8(const void *q, const int64_t q_strides[3], const void *k_cache, const void *v_cache,
                        const float *k_scale, const float *v_scale, const int64_t cache_strides[3],
                        const int32_t *positions, const int32_t *new_lens, int64_t max_seq_len,
                        const int32_t *page_table, int64_t max_pages, int64_t num_pages, void *out,
                        const int64_t out_strides[3], int64_t batch, int64_t num_new, int64_t num_q_heads,
                        int64_t num_kv_heads, int64_t head_dim, int64_t page_size, float sm_scale,
                        tt_stream_t stream) {
  return prefill_common(tt::CacheKind::kFP8, q, q_strides, k_cache, v_cache, k_scale, v_scale, cache_strides,
                        positions, new_lens, max_seq_len, page_table, max_pages, num_pages, out, out_strides, batch,
                        num_new, num_q_heads, num_kv_heads, head_dim, page_size, sm_scale, stream);
}

int tt_gqa_decode_attn_bf16(const void *q, const int64_t q_strides[2], const void *k_cache, const void *v_cache,
                            const int64_t cache_strides[3], const int32_t *seq_lens, int64_t max_seq_len,
                            const int32_t *page_table, int64_t max_pages, int64_t num_pages, void *out,
                            const int64_t out_strides[2], int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                            int64_t head_dim, int64_t page_size, float sm_scale, int64_t split_tokens,
                            const int32_t *length_order, void *workspace, size_t workspace_bytes,
                            tt_stream_t stream) {
  return decode_common(tt::CacheKind::kBF16, q, q_strides, k_cache, v_cache, nullptr, nullptr, cache_strides,
                       seq_lens, max_seq_len, page_table, max_pages, num_pages, out, out_strides, batch, num_q_heads,
                       num_kv_heads, head_dim, page_size, sm_scale, split_tokens, workspace, workspace_bytes, stream,
                       nullptr, false, nullptr, 0, length_order);
}

int tt_gqa_decode_attn_fp8(const void *q, const int64_t q_strides[2], const void *k_cache, const void *v_cache,
                           const float *k_scale, const float *v_scale, const int64_t cache_strides[3],
                           const int32_t *seq_lens, int64_t max_seq_len, const int32_t *page_table,
                           int64_t max_pages, int64_t num_pages, void *out, const int64_t out_strides[2],
                           int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                           int64_t page_size, float sm_scale, int64_t split_tokens, const int32_t *length_order,
                           void *workspace, size_t workspace_bytes, tt_stream_t stream) {
  return decode_common(tt::CacheKind::kFP8, q, q_strides, k_cache, v_cache, k_scale, v_scale, cache_strides,
                       seq_lens, max_seq_len, page_table, max_pages, num_pages, out, out_strides, batch, num_q_heads,
                       num_kv_heads, head_dim, page_size, sm_scale, split_tokens, workspace, workspace_bytes, stream,
                       nullptr, false, nullptr, 0, length_order);
}

int tt_gqa_decode_attn_f32(const void *q, const int64_t q_strides[2], const void *k_cache, const void *v_cache,
                           const int64_t cache_strides[3], const int32_t *seq_lens, int64_t max_seq_len,
                           const int32_t *page_table, int64_t max_pages, int64_t num_pages, void *out,
                           const int64_t out_strides[2], int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                           int64_t head_dim, int64_t page_size, float sm_scale, int64_t split_tokens,
                           void *workspace, size_t workspace_bytes, tt_stream_t stream) {
  return decode_common(tt::CacheKind::kF32, q, q_strides, k_cache, v_cache, nullptr, nullptr, cache_strides, seq_lens,
                       max_seq_len, page_table, max_pages, num_pages, out, out_strides, batch, num_q_heads,
                       num_kv_heads, head_dim, page_size, sm_scale, split_tokens, workspace, workspace_bytes, stream);
}

int tt_rows_attn_bf16(const void *q, const int64_t q_strides[2], const void *k_cache, const void *v_cache,
                      const int64_t cache_strides[3], const int32_t *seq_of_row, const int32_t *row_lens,
                      int64_t max_row_len, const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                      int64_t num_seqs, void *out, const int64_t out_strides[2], int64_t rows, int64_t num_q_heads,
                      int64_t num_kv_heads, int64_t head_dim, int64_t page_size, float sm_scale, void *workspace,
                      size_t workspace_bytes, tt_stream_t stream) {
  TT_CHECK(seq_of_row != nullptr, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  return decode_common(tt::CacheKind::kBF16, q, q_strides, k_cache, v_cache, nullptr, nullptr, cache_strides, row_lens,
                       max_row_len, page_table, max_pages, num_pages, out, out_strides, rows, num_q_heads,
                       num_kv_heads, head_dim, page_size, sm_scale, 0, workspace, workspace_bytes, stream, nullptr,
                       false, seq_of_row, num_seqs);
}

int tt_rows_attn_fp8(const void *q, const int64_t q_strides[2], const void *k_cache, const void *v_cache,
                     const float *k_scale, const float *v_scale, const int64_t cache_strides[3],
                     const int32_t *seq_of_row, const int32_t *row_lens, int64_t max_row_len,
                     const int32_t *page_table, int64_t max_pages, int64_t num_pages, int64_t num_seqs, void *out,
                     const int64_t out_strides[2], int64_t rows, int64_t num_q_heads, int64_t num_kv_heads,
                     int64_t head_dim, int64_t page_size, float sm_scale, void *workspace, size_t workspace_bytes,
                     tt_stream_t stream) {
  TT_CHECK(seq_of_row != nullptr, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  return decode_common(tt::CacheKind::kFP8, q, q_strides, k_cache, v_cache, k_scale, v_scale, cache_strides, row_lens,
                       max_row_len, page_table, max_pages, num_pages, out, out_strides, rows, num_q_heads,
                       num_kv_heads, head_dim, page_size, sm_scale, 0, workspace, workspace_bytes, stream, nullptr,
                       false, seq_of_row, num_seqs);
}

int tt_rows_attn_f32(const void *q, const int64_t q_strides[2], const void *k_cache, const void *v_cache,
                     const int64_t cache_strides[3], const int32_t *seq_of_row, const int32_t *row_lens,
                     int64_t max_row_len, const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                     int64_t num_seqs, void *out, const int64_t out_strides[2], int64_t rows, int64_t num_q_heads,
                     int64_t num_kv_heads, int64_t head_dim, int64_t page_size, float sm_scale, void *workspace,
                     size_t workspace_bytes, tt_stream_t stream) {
  TT_CHECK(seq_of_row != nullptr, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  return decode_common(tt::CacheKind::kF32, q, q_strides, k_cache, v_cache, nullptr, nullptr, cache_strides, row_lens,
                       max_row_len, page_table, max_pages, num_pages, out, out_strides, rows, num_q_heads,
                       num_kv_heads, head_dim, page_size, sm_scale, 0, workspace, workspace_bytes, stream, nullptr,
                       false, seq_of_row, num_seqs);
}

int64_t tt_decode_split_tokens(int64_t batch, int64_t num_kv_heads, int64_t max_seq_len) {
  return tt::auto_split_tokens(batch, num_kv_heads, max_seq_len);
}

int64_t tt_decode_pick_split(const int32_t *seq_lens_host, int64_t batch, int64_t num_kv_heads, int64_t head_dim,
                             int32_t fp8_cache) {
  if (seq_lens_host == nullptr || batch <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
  const tt::CacheKind kind = fp8_cache ? tt::CacheKind::kFP8 : tt::CacheKind::kBF16;
  const int tile = tt::tile_head_dim(head_dim, kind);
  if (tile == 0) return 0;
  bool equal = true;
  for (int64_t b = 1; b < batch && equal; ++b) equal = seq_lens_host[b] == seq_lens_host[0];
  if (equal) return (batch * num_kv_heads) % tt::segment_round(tile) == 0 ? tt::kSplitPerSegment : 0;
  // The paired partition: one round of the GPU's CUs (one workgroup per CU,
  // two at 4 waves a workgroup), its workgroups' work (two segments' tiles and
  // start-up positions) within kPairedSlack of the mean. Measured against the
  // balanced partition (ragged, fused step): C5 layer (pairs 1.034 of the
  // mean) 35.2 -> 30.6 us, C3 (1.049) 386 -> 381 us, C4 (1.064) 747 -> 749 us.
  constexpr double kPairedSlack = 1.06;
  if (batch > tt::kMaxPairedBatch || (batch + 1) / 2 * num_kv_heads % tt::device_cu_count() != 0) return 0;
  if (tt::paired_lds_bytes(tile, fp8_cache != 0, true, 16) == 0) return 0;  // fits every GQA group up to 16
  int64_t lines[tt::kMaxPairedBatch];
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t L = seq_lens_host[b] > 0 ? seq_lens_host[b] : 0;
    lines[b] = L > 0 ? (L + tt::kTileTokens - 1) / tt::kTileTokens + tt::kStreamSegCost : 0;
  }
  std::sort(lines, lines + batch);
  int64_t worst = 0, total = 0;
  for (int64_t p = 0; p < (batch + 1) / 2; ++p) {
    const int64_t w = lines[batch - 1 - p] + (batch - 1 - p != p ? lines[p] : 0);
    worst = std::max(worst, w);
    total += w;
  }
  if (total == 0) return 0;
  const double mean = (double)total / (double)((batch + 1) / 2);
  return (double)worst <= kPairedSlack * mean ? tt::kSplitPaired : 0;
}

size_t tt_decode_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                 int64_t max_seq_len, int64_t split_tokens) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
  const int64_t split = resolve_split(split_tokens, batch, num_kv_heads, max_seq_len);
  if (split <= 0) return 0;
  const size_t fixed = workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, max_seq_len, split);
  if (split_tokens != 0) return fixed;
  // 0 serves every cache dtype: the balanced layout (bf16, fp8) or the automatic split (fp32)
  const size_t bal = balanced_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim);
  return bal > fixed ? bal : fixed;
}

int tt_linear_splitk_bf16(const void *x, int64_t ldx, const void *weight, int64_t ldw, float *partials, int64_t m,
                          int64_t n, int64_t k, int64_t k_chunk, tt_stream_t stream) {
  return linear_common(x, ldx, weight, ldw, 0, partials, m, n, k, k_chunk, stream);
}

int tt_linear_splitk_packed_bf16(const void *x, int64_t ldx, const void *weight_packed, float *partials, int64_t m,
                                 int64_t n, int64_t k, int64_t k_chunk, tt_stream_t stream) {
  return linear_common(x, ldx, weight_packed, k, 1, partials, m, n, k, k_chunk, stream);
}



int tt_splitk_reduce_bf16(const float *partials, int64_t splits, int64_t m, int64_t n, void *y, tt_stream_t stream) {
  TT_CHECK(partials && y, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(splits >= 1 && splits <= 4096 && m >= 0 && n > 0, TT_ERR_INVALID_ARGUMENT, "bad reduce shape");
  TT_CHECK((m * n) % 4 == 0, TT_ERR_UNSUPPORTED, "M * N must be a multiple of 4");
  TT_CHECK(aligned(partials, 16) && aligned(y, 8), TT_ERR_INVALID_ARGUMENT, "partials / y misaligned");
  if (m == 0) return ok();
  (void)hipGetLastError();
  return from_hip(tt::launch_reduce_bf16(partials, (int)splits, m * n, static_cast<uint16_t *>(y), (hipStream_t)stream),
                  "reduce launch");
}

int tt_add_rmsnorm_bf16(float *x, const float *partials, int64_t splits, const float *weight, float eps, void *y,
                        int64_t m, int64_t c, tt_stream_t stream) {
  TT_CHECK(x && weight && y, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(m >= 0 && m <= 0x7fffffff, TT_ERR_INVALID_ARGUMENT, "bad row count");
  TT_CHECK(c % 4 == 0 && c >= 4 && c <= 8192, TT_ERR_UNSUPPORTED,
           "hidden size must be a multiple of 4 in [4, 8192], got %lld", (long long)c);
  TT_CHECK(partials == nullptr || (splits >= 1 && splits <= 4096), TT_ERR_INVALID_ARGUMENT, "bad split count");
  TT_CHECK(aligned(x, 16) && aligned(weight, 16) && aligned(y, 8) && (partials == nullptr || aligned(partials, 16)),
           TT_ERR_INVALID_ARGUMENT, "x / weight / partials must be 16-byte aligned, y 8-byte aligned");
  if (m == 0) return ok();
  (void)hipGetLastError();
  return from_hip(tt::launch_add_rmsnorm(x, partials, partials ? (int)splits : 0, (int)m, (int)c, weight, eps,
                                         static_cast<uint16_t *>(y), (hipStream_t)stream),
                  "add_rmsnorm launch");
}

int tt_silu_mul_bf16(const float *partials, int64_t splits, int64_t m, int64_t inter, void *y, tt_stream_t stream) {
  TT_CHECK(partials && y, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(splits >= 1 && splits <= 4096 && m >= 0 && inter > 0, TT_ERR_INVALID_ARGUMENT, "bad shape");
  TT_CHECK(inter % 4 == 0 && inter < ((int64_t)1 << 30), TT_ERR_UNSUPPORTED, "intermediate size must be a multiple of 4");
  TT_CHECK(aligned(partials, 16) && aligned(y, 8), TT_ERR_INVALID_ARGUMENT, "partials / y misaligned");
  if (m == 0) return ok();
  (void)hipGetLastError();
  return from_hip(tt::launch_silu_mul(partials, (int)splits, (int)m, (int)inter, static_cast<uint16_t *>(y),
                                      (hipStream_t)stream),
                  "silu_mul launch");
}

int tt_swiglu_gemm_supported(int64_t k, int64_t inter) { return tt::swiglu_gemm_supported(k, inter) ? 1 : 0; }

int tt_linear_swiglu_packed_bf16(const void *x, int64_t ldx, const void *weight_packed, void *y, int64_t ldy,
                                 int64_t m, int64_t inter, int64_t k, tt_stream_t stream) {
  TT_CHECK(x && weight_packed && y, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(m >= 0 && m <= 65535 * 64 && inter > 0 && k > 0, TT_ERR_INVALID_ARGUMENT, "bad GEMM shape");
  TT_CHECK(tt::swiglu_gemm_supported(k, inter), TT_ERR_UNSUPPORTED,
           "the fused gate|up + SwiGLU GEMM takes K 768, 1024 or 2048 and I a multiple of 16 or 24 (K %lld, I %lld)", (long long)k,
           (long long)inter);
  TT_CHECK(inter < ((int64_t)1 << 30), TT_ERR_UNSUPPORTED, "intermediate size too large");
  TT_CHECK(ldx >= k && ldx % 8 == 0 && ldy >= inter && ldy % 4 == 0, TT_ERR_INVALID_ARGUMENT,
           "ldx must be >= K and a multiple of 8, ldy >= I and a multiple of 4");
  TT_CHECK(ldx < ((int64_t)1 << 24), TT_ERR_UNSUPPORTED, "x row stride too large");
  TT_CHECK(aligned(x, 16) && aligned(weight_packed, 16) && aligned(y, 8), TT_ERR_INVALID_ARGUMENT,
           "x and weight must be 16-byte aligned, y 8-byte aligned");
  if (m == 0) return ok();
  tt::SwigluGemmArgs a{};
  a.x = static_cast<const uint16_t *>(x);
  a.ldx = ldx;
  a.w = static_cast<const uint16_t *>(weight_packed);
  a.out = static_cast<uint16_t *>(y);
  a.ldo = ldy;
  a.M = (int)m;
  a.I = (int)inter;
  a.K = (int)k;
  (void)hipGetLastError();
  return from_hip(tt::launch_swiglu_gemm(a, (hipStream_t)stream), "linear_swiglu launch");
}

int tt_add_rmsnorm_rows_bf16(float *x, const void *a, int64_t lda, const float *weight, float eps, void *y, int64_t m,
                             int64_t c, tt_stream_t stream) {
  TT_CHECK(x && weight && y, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(m >= 0 && m <= 0x7fffffff, TT_ERR_INVALID_ARGUMENT, "bad row count");
  TT_CHECK(c % 4 == 0 && c >= 4 && c <= 8192, TT_ERR_UNSUPPORTED,
           "hidden size must be a multiple of 4 in [4, 8192], got %lld", (long long)c);
  TT_CHECK(a == nullptr || (lda >= c && lda % 4 == 0), TT_ERR_INVALID_ARGUMENT, "addend row stride must be >= C and a multiple of 4");
  TT_CHECK(aligned(x, 16) && aligned(weight, 16) && aligned(y, 8) && (a == nullptr || aligned(a, 8)),
           TT_ERR_INVALID_ARGUMENT, "x / weight must be 16-byte aligned, y / addend 8-byte aligned");
  if (m == 0) return ok();
  (void)hipGetLastError();
  return from_hip(tt::launch_add_rmsnorm_rows(x, static_cast<const uint16_t *>(a), lda, (int)m, (int)c, weight, eps,
                                              static_cast<uint16_t *>(y), (hipStream_t)stream),
                  "add_rmsnorm_rows launch");
}

int tt_silu_mul_rows_bf16(const void *g, int64_t ldg, const void *u, int64_t ldu, int64_t m, int64_t inter, void *y,
                          tt_stream_t stream) {
  TT_CHECK(g && u && y, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(m >= 0 && inter > 0 && ldg >= inter && ldu >= inter, TT_ERR_INVALID_ARGUMENT, "bad shape");
  TT_CHECK(inter % 4 == 0 && ldg % 4 == 0 && ldu % 4 == 0 && inter < ((int64_t)1 << 30), TT_ERR_UNSUPPORTED,
           "intermediate size and row strides must be multiples of 4");
  TT_CHECK(m * inter < ((int64_t)1 << 40), TT_ERR_UNSUPPORTED, "too many elements");
  TT_CHECK(aligned(g, 8) && aligned(u, 8) && aligned(y, 8), TT_ERR_INVALID_ARGUMENT, "g / u / y must be 8-byte aligned");
  if (m == 0) return ok();
  (void)hipGetLastError();
  return from_hip(tt::launch_silu_mul_rows(static_cast<const uint16_t *>(g), ldg, static_cast<const uint16_t *>(u), ldu,
                                           m, (int)inter, static_cast<uint16_t *>(y), (hipStream_t)stream),
                  "silu_mul_rows launch");
}

int tt_decode_attn_append_bf16(const void *q_in, const int64_t q_in_strides[2], const void *k_in,
                               const int64_t k_in_strides[2], const void *v_in, const int64_t v_in_strides[2],
                               int64_t splits, int64_t split_stride, const void *rope_table, int64_t rope_table_len,
                               const int32_t *positions, int32_t *lens_out, int64_t max_seq_len,
                               const int32_t *page_table, int64_t max_pages, int64_t num_pages, void *k_cache,
                               void *v_cache, const int64_t cache_strides[3], int64_t capacity, void *out,
                               const int64_t out_strides[2], int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                               int64_t head_dim, int64_t page_size, float sm_scale, int64_t split_tokens,
                               const int32_t *length_order, void *workspace, size_t workspace_bytes,
                               tt_stream_t stream) {
  return decode_append_common(tt::CacheKind::kBF16, q_in, q_in_strides, k_in, k_in_strides, v_in, v_in_strides,
                              splits, split_stride, rope_table, rope_table_len, positions, lens_out, max_seq_len,
                              page_table, max_pages, num_pages, k_cache, v_cache, nullptr, nullptr, cache_strides,
                              capacity, out, out_strides, batch, num_q_heads, num_kv_heads, head_dim, page_size,
                              sm_scale, split_tokens, length_order, workspace, workspace_bytes, stream);
}

int tt_decode_attn_append_fp8(const void *q_in, const int64_t q_in_strides[2], const void *k_in,
                              const int64_t k_in_strides[2], const void *v_in, const int64_t v_in_strides[2],
                              int64_t splits, int64_t split_stride, const void *rope_table, int64_t rope_table_len,
                              const int32_t *positions, int32_t *lens_out, int64_t max_seq_len,
                              const int32_t *page_table, int64_t max_pages, int64_t num_pages, void *k_cache,
                              void *v_cache, float *k_scale, float *v_scale, const int64_t cache_strides[3],
                              int64_t capacity, void *out, const int64_t out_strides[2], int64_t batch,
                              int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                              float sm_scale, int64_t split_tokens, const int32_t *length_order, void *workspace,
                              size_t workspace_bytes, tt_stream_t stream) {
  return decode_append_common(tt::CacheKind::kFP8, q_in, q_in_strides, k_in, k_in_strides, v_in, v_in_strides,
                              splits, split_stride, rope_table, rope_table_len, positions, lens_out, max_seq_len,
                              page_table, max_pages, num_pages, k_cache, v_cache, k_scale, v_scale, cache_strides,
                              capacity, out, out_strides, batch, num_q_heads, num_kv_heads, head_dim, page_size,
                              sm_scale, split_tokens, length_order, workspace, workspace_bytes, stream);
}

int tt_decode_attn_append_bf16_noalloc(const void *q_in, const int64_t q_in_strides[2], const void *k_in,
                                       const int64_t k_in_strides[2], const void *v_in, const int64_t v_in_strides[2],
                                       int64_t splits, int64_t split_stride, const void *rope_table,
                                       int64_t rope_table_len, const int32_t *positions, int32_t *lens_out,
                                       int64_t max_seq_len, const int32_t *page_table, int64_t max_pages,
                                       int64_t num_pages, void *k_cache, void *v_cache, const int64_t cache_strides[3],
                                       int64_t capacity, void *out, const int64_t out_strides[2], int64_t batch,
                                       int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                       float sm_scale, tt_stream_t stream) {
  void *ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != TT_OK) return rc;
  return decode_append_common(tt::CacheKind::kBF16, q_in, q_in_strides, k_in, k_in_strides, v_in, v_in_strides,
                              splits, split_stride, rope_table, rope_table_len, positions, lens_out, max_seq_len,
                              page_table, max_pages, num_pages, k_cache, v_cache, nullptr, nullptr, cache_strides,
                              capacity, out, out_strides, batch, num_q_heads, num_kv_heads, head_dim, page_size,
                              sm_scale, 0, nullptr, ws, kScratchBytes, stream, /*exact_slots=*/true);
}

int tt_decode_layers_bf16(const tt_decode_layer_t *layers, int64_t num_layers, int64_t max_seq_len,
                          tt_stream_t stream) {
  TT_CHECK(layers != nullptr || num_layers == 0, TT_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
  TT_CHECK(num_layers >= 0, TT_ERR_INVALID_ARGUMENT, "num_layers must be >= 0");
  for (int64_t i = 0; i < num_layers; ++i) {
    const tt_decode_layer_t &L = layers[i];
    const int64_t B = L.batch, C = L.hidden, I = L.intermediate, Hq = L.num_q_heads, Hkv = L.num_kv_heads;
    const int64_t D = L.head_dim, Nqkv = (Hq + 2 * Hkv) * D;
    int rc = TT_OK;
    auto step = [&](int status, const char *what) {
      if (status != TT_OK && rc == TT_OK) {
        rc = status;
        const std::string msg = g_last_error;  // prefix the step that failed
        fail(status, "layer %lld, %s: %s", (long long)i, what, msg.c_str());
      }
      return rc == TT_OK;
    };
    TT_CHECK(L.kc_qkv > 0 && L.kc_o > 0 && L.kc_down > 0 && L.kc_gu >= 0, TT_ERR_INVALID_ARGUMENT,
             "layer %lld: bad k_chunk", (long long)i);
    // q|k|v projection: split-K partials read by the attention step
    if (!step(tt_linear_splitk_packed_bf16(L.h, C, L.w_qkv, L.partials, B, Nqkv, C, L.kc_qkv, stream), "q|k|v"))
      return rc;
    const int64_t S = C / L.kc_qkv;
    const int64_t pst[2] = {Nqkv, D};
    const int64_t ost[2] = {Hq * D, D};
    const char *base = reinterpret_cast<const char *>(L.partials);
    const void *q_in = base, *k_in = base + Hq * D * 4, *v_in = base + (Hq + Hkv) * D * 4;
    const int attn =
        L.fp8_cache
            ? tt_decode_attn_append_fp8(q_in, pst, k_in, pst, v_in, pst, S, B * Nqkv, L.rope_table, L.rope_table_len,
                                        L.positions, L.lens_out, max_seq_len, L.page_table, L.max_pages, L.num_pages,
                                        L.k_cache, L.v_cache, L.k_scale, L.v_scale, L.cache_strides, L.capacity,
                                        L.attn_out, ost, B, Hq, Hkv, D, L.page_size, L.sm_scale, L.split_tokens,
                                        L.length_order, L.workspace, L.workspace_bytes, stream)
            : tt_decode_attn_append_bf16(q_in, pst, k_in, pst, v_in, pst, S, B * Nqkv, L.rope_table, L.rope_table_len,
                                         L.positions, L.lens_out, max_seq_len, L.page_table, L.max_pages, L.num_pages,
                                         L.k_cache, L.v_cache, L.cache_strides, L.capacity, L.attn_out, ost, B, Hq,
                                         Hkv, D, L.page_size, L.sm_scale, L.split_tokens, L.length_order, L.workspace,
                                         L.workspace_bytes, stream);
    if (!step(attn, "attention")) return rc;
    if (!step(tt_linear_splitk_packed_bf16(L.attn_out, Hq * D, L.w_o, L.partials, B, C, Hq * D, L.kc_o, stream),
              "c_proj"))
      return rc;
    if (!step(tt_add_rmsnorm_bf16(L.x, L.partials, (Hq * D) / L.kc_o, L.ln2_weight, L.eps, L.h, B, C, stream),
              "residual + norm 2"))
      return rc;
    if (L.kc_gu == 0) {
      if (!step(tt_linear_swiglu_packed_bf16(L.h, C, L.w_gu, L.act, I, B, I, C, stream), "gate|up + SwiGLU"))
        return rc;
    } else {
      if (!step(tt_linear_splitk_packed_bf16(L.h, C, L.w_gu, L.partials, B, 2 * I, C, L.kc_gu, stream), "gate|up"))
        return rc;
      if (!step(tt_silu_mul_bf16(L.partials, C / L.kc_gu, B, I, L.act, stream), "SwiGLU")) return rc;
    }
    if (!step(tt_linear_splitk_packed_bf16(L.act, I, L.w_down, L.partials, B, C, I, L.kc_down, stream), "down"))
      return rc;
    if (!step(tt_add_rmsnorm_bf16(L.x, L.partials, I / L.kc_down, L.next_norm_weight, L.eps, L.h, B, C, stream),
              "residual + next norm"))
      return rc;
  }
  return ok();
}

size_t tt_sample_workspace_bytes(int64_t m, int64_t vocab, int64_t top_k) {
  if (m <= 0 || vocab <= 0) return 0;
  const int chunks = tt::sample_cand_chunks(m, vocab, top_k > 0 && top_k < vocab ? top_k : 0, false);
  return (size_t)m * chunks * sizeof(tt::CandRecord);
}

int tt_sample_bf16(const void *logits, int64_t ld, int64_t m, int64_t vocab, float temperature, int64_t top_k,
                   float top_p, uint64_t seed, uint64_t offset, int64_t *tokens, float *token_logprob,
                   float *logprobs, int64_t ld_logprobs, void *workspace, size_t workspace_bytes,
                   tt_stream_t stream) {
  return sample_common(false, logits, ld, m, vocab, temperature, top_k, top_p, seed, offset, tokens, token_logprob,
                       logprobs, ld_logprobs, workspace, workspace_bytes, stream);
}

int tt_sample_f32(const float *logits, int64_t ld, int64_t m, int64_t vocab, float temperature, int64_t top_k,
                  float top_p, uint64_t seed, uint64_t offset, int64_t *tokens, float *token_logprob,
                  float *logprobs, int64_t ld_logprobs, void *workspace, size_t workspace_bytes,
                  tt_stream_t stream) {
  return sample_common(true, logits, ld, m, vocab, temperature, top_k, top_p, seed, offset, tokens, token_logprob,
                       logprobs, ld_logprobs, workspace, workspace_bytes, stream);
}

}  // extern "C"
