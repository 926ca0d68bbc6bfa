// Byte-moving kernels of the decode path: the paged KV cache write and the
// row gathers (embedding lookup, sampled-row gather). All are HBM-bound bit
// copies done with 16-byte vector loads/stores; results are bit-exact.
#include "common.h"

namespace sid {
namespace {

// One workgroup row per token. A token's K (or V) row is HKV*D bf16 =
// 2 KiB for Qwen3 shapes, i.e. 128 16-byte vectors; thread i copies vector i
// of K and of V. Slots are validated on the device: <0 is padding (skipped
// as in sid/csrc/flash_decode.cu:285), >= num_slots would be out of bounds.
__global__ void __launch_bounds__(256) reshape_and_cache_kernel(
    const uint4* __restrict__ k, const uint4* __restrict__ v, uint4* __restrict__ k_cache,
    uint4* __restrict__ v_cache, const int64_t* __restrict__ slot_mapping, int64_t num_tokens,
    int vec_per_row, int64_t num_slots) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.y + threadIdx.y;
  if (t >= num_tokens) return;
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= num_slots) return;
  const uint4* ks = k + t * vec_per_row;
  const uint4* vs = v + t * vec_per_row;
  uint4* kd = k_cache + slot * vec_per_row;
  uint4* vd = v_cache + slot * vec_per_row;
  for (int c = threadIdx.x; c < vec_per_row; c += blockDim.x) {
    const uint4 kk = ks[c];
    const uint4 vv = vs[c];
    kd[c] = kk;
    vd[c] = vv;
  }
}

__global__ void __launch_bounds__(256) gather_rows_kernel(
    const uint4* __restrict__ table, const int64_t* __restrict__ idx, uint4* __restrict__ out,
    int64_t n, int64_t vec_per_row, int64_t table_rows) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.y + threadIdx.y;
  if (r >= n) return;
  const int64_t src = idx[r];
  uint4* dst = out + r * vec_per_row;
  if (src < 0 || src >= table_rows) {
    for (int64_t c = threadIdx.x; c < vec_per_row; c += blockDim.x) dst[c] = make_uint4(0, 0, 0, 0);
    return;
  }
  const uint4* s = table + src * vec_per_row;
  for (int64_t c = threadIdx.x; c < vec_per_row; c += blockDim.x) dst[c] = s[c];
}


// Decode-batch construction on the device, over page tables. Request b owns
// row rows[b] of the block table [num_rows, max_pages] (int32 page ids; a page
// holds `page_size` = 1 << page_shift consecutive pool slots) and has
// L = kv_indptr[b+1] - kv_indptr[b] positions, the last of which is the token
// decoded now; its slot new_slots[b] was chosen on the host. Position i < L-1
// lives in slot table[i >> shift] * page_size + (i & mask). When the new token
// opens a page (position L-1 is a page's first), its page id enters the table
// for later steps; no thread of this launch reads that entry (every earlier
// position lies in an earlier page), so there is no intra-launch dependency.
// Consecutive threads take consecutive positions: a wave reads one or a few
// table entries (broadcast) and writes 256 contiguous bytes of kv_indices.
__global__ void __launch_bounds__(256) build_paged_decode_indices_kernel(
    int32_t* __restrict__ tables, int64_t max_pages, int64_t num_rows, int page_shift,
    const int64_t* __restrict__ rows, const int64_t* __restrict__ new_slots,
    const int32_t* __restrict__ kv_indptr, int32_t* __restrict__ kv_indices) {
  const int b = blockIdx.x;
  const int64_t row = rows[b];
  const int start = kv_indptr[b];
  const int len = kv_indptr[b + 1] - start;
  if (row < 0 || row >= num_rows || len <= 0 || ((len - 1) >> page_shift) >= max_pages) return;
  int32_t* table = tables + row * max_pages;
  const int32_t mask = (1 << page_shift) - 1;
  const int last = len - 1;
  // Eight positions per thread per pass, their table entries loaded together (one round trip
  // per 2048 positions instead of one per 256).
  constexpr int U = 8;
  for (int i0 = threadIdx.x; i0 < last; i0 += 256 * U) {
    int32_t pg[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + 256 * u;
      pg[u] = i < last ? table[i >> page_shift] : 0;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + 256 * u;
      if (i < last) kv_indices[start + i] = (pg[u] << page_shift) | (i & mask);
    }
  }
  if (threadIdx.x == 0) {
    const int32_t slot = static_cast<int32_t>(new_slots[b]);
    kv_indices[start + last] = slot;
    if ((last & mask) == 0) table[last >> page_shift] = slot >> page_shift;
  }
}

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int sid_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                                     const int64_t* slot_mapping, int64_t num_tokens,
                                     int num_kv_heads, int head_dim, int64_t num_slots,
                                     void* stream) {
  SID_REQUIRE(num_tokens >= 0, "reshape_and_cache: negative token count %lld",
              (long long)num_tokens);
  if (num_tokens == 0) return SID_OK;
  SID_REQUIRE(k && v && k_cache && v_cache && slot_mapping, "reshape_and_cache: null pointer");
  SID_REQUIRE(num_kv_heads > 0 && head_dim > 0 && (num_kv_heads * head_dim) % 8 == 0,
              "reshape_and_cache: row of %d x %d bf16 is not a whole number of 16-byte vectors",
              num_kv_heads, head_dim);
  SID_REQUIRE(num_slots > 0, "reshape_and_cache: empty pool");
  const int vec_per_row = num_kv_heads * head_dim / 8;
  // Threads per row: up to 128 (one 16-byte vector each), rows per block fill 256 threads.
  const int tx = vec_per_row >= 128 ? 128 : (vec_per_row >= 64 ? 64 : 32);
  const int ty = 256 / tx;
  const dim3 block(tx, ty);
  const int64_t blocks = (num_tokens + ty - 1) / ty;
  SID_REQUIRE(blocks < (1ll << 31), "reshape_and_cache: too many tokens");
  hipLaunchKernelGGL(reshape_and_cache_kernel, dim3((unsigned)blocks), block, 0,
                     (hipStream_t)stream, (const uint4*)k, (const uint4*)v, (uint4*)k_cache,
                     (uint4*)v_cache, slot_mapping, num_tokens, vec_per_row, num_slots);
  return check_launch("reshape_and_cache");
}

extern "C" int sid_gather_rows(const void* table, const int64_t* idx, void* out, int64_t n,
                               int64_t row_elems, int64_t table_rows, void* stream) {
  SID_REQUIRE(n >= 0, "gather_rows: negative row count");
  if (n == 0) return SID_OK;
  SID_REQUIRE(table && idx && out, "gather_rows: null pointer");
  SID_REQUIRE(row_elems > 0 && row_elems % 8 == 0,
              "gather_rows: row of %lld bf16 is not a whole number of 16-byte vectors",
              (long long)row_elems);
  const int64_t vec = row_elems / 8;
  const int tx = vec >= 128 ? 128 : (vec >= 64 ? 64 : 32);
  const int ty = 256 / tx;
  const int64_t blocks = (n + ty - 1) / ty;
  SID_REQUIRE(blocks < (1ll << 31), "gather_rows: too many rows");
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)blocks), dim3(tx, ty), 0,
                     (hipStream_t)stream, (const uint4*)table, idx, (uint4*)out, n, vec,
                     table_rows);
  return check_launch("gather_rows");
}

extern "C" int sid_build_paged_decode_indices(int32_t* block_tables, int64_t max_pages,
                                              int64_t num_rows, int page_size,
                                              const int64_t* rows, const int64_t* new_slots,
                                              const int32_t* kv_indptr, int32_t* kv_indices,
                                              int batch, void* stream) {
  SID_REQUIRE(batch >= 0, "build_paged_decode_indices: negative batch");
  if (batch == 0) return SID_OK;
  SID_REQUIRE(block_tables && rows && new_slots && kv_indptr && kv_indices,
              "build_paged_decode_indices: null pointer");
  SID_REQUIRE(max_pages > 0 && num_rows > 0, "build_paged_decode_indices: empty table");
  SID_REQUIRE(page_size > 0 && (page_size & (page_size - 1)) == 0 && page_size <= (1 << 20),
              "build_paged_decode_indices: page_size %d is not a power of two", page_size);
  int shift = 0;
  while ((1 << shift) < page_size) ++shift;
  hipLaunchKernelGGL(build_paged_decode_indices_kernel, dim3(batch), dim3(256), 0,
                     (hipStream_t)stream, block_tables, max_pages, num_rows, shift, rows,
                     new_slots, kv_indptr, kv_indices);
  return check_launch("build_paged_decode_indices");
}
