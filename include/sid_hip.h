/*
 * sid_hip.h — C-ABI of the MI355X (gfx950) decode hot path of sid.
 *
 * Every entry point takes raw device pointers, sizes and a hipStream_t passed
 * as `void* stream` (NULL = the default stream), launches asynchronously on
 * that stream, allocates nothing and returns SID_OK or an error code; the
 * message for the last error on the calling thread is sid_last_error().
 * bf16 tensors are passed as `void*` (raw 16-bit bf16 bits), row-major and
 * contiguous. Shapes use the reference's names: B requests, T tokens,
 * HQ = 16 query heads, HKV = 8 KV heads, D = 128 head dim, S pool slots.
 *
 * Reference interfaces replaced (paths relative to the sid repository):
 *   sid/csrc/flash_decode.cu         pybind module `sid_flash_decode`
 *   sid/kernels/extend_attention.py  Triton extend attention
 *   sid/kernels/rmsnorm.py           Triton RMSNorm kernels
 *   sid/kernels/rope.py              Triton RoPE kernel
 *   sid/kernels/matmul_persistent.py Triton persistent GEMM / F.linear
 *   sid/model/qwen3.py               torch glue (embedding, silu*up, row gather)
 *   sid/engine/sampler.py            greedy argmax
 */
#ifndef SID_HIP_H_
#define SID_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SID_OK 0
#define SID_ERR_INVALID 1 /* bad argument: shape, size, null pointer */
#define SID_ERR_LAUNCH 2  /* the HIP runtime rejected a launch */

/* Message describing the last non-SID_OK return on this thread ("" if none). */
const char* sid_last_error(void);

/* ABI version of this library (bumped on any signature or precondition change). */
int sid_abi_version(void);

/*
 * Scatter new K/V rows into the paged KV pool: k_cache[slot[t]] = k[t],
 * v_cache[slot[t]] = v[t]. k, v: bf16 [T, HKV, D]; k_cache, v_cache: bf16
 * [S, HKV, D]; slot_mapping: int64 [T]. Slots < 0 are skipped (padding);
 * slots >= S are skipped too, so a bad mapping cannot write out of bounds.
 * Replaces reshape_and_cache, sid/csrc/flash_decode.cu:378-406 (kernel
 * :275-296).
 */
int sid_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                          const int64_t* slot_mapping, int64_t num_tokens, int num_kv_heads,
                          int head_dim, int64_t num_slots, void* stream);

/*
 * Split-KV paged decode attention (stage 1 partial softmax per KV split,
 * stage 2 log-sum-exp merge in fixed split order). q, o: bf16 [B, HQ, D];
 * k_cache, v_cache: bf16 [S, HKV, D]; kv_indptr int32 [B+1]; kv_indices int32
 * [kv_indptr[B]] (pool slot of every position, in order); num_splits int32
 * [B]; part_o fp32 [part_batch, HQ, part_stride, D]; part_lse fp32
 * [part_batch, HQ, part_stride]. fixed_split_size > 0 gives fixed-size splits
 * (batch-invariant mode), 0 the heuristic geometry
 * ceil(ceil(len / n) / 32) * 32. Requires HKV == 8, HQ == 16, D == 128
 * (the Qwen3 attention shape), part_batch >= B, part_stride >= max_splits >=
 * 1. Slots outside [0, S) read slot 0. When max_splits == 1 the workspace is
 * not touched. Equals sid_flash_decode_segments_fwd with segment_size 0 and
 * grid_slots = max_splits.
 * Replaces flash_decode_fwd, sid/csrc/flash_decode.cu:307-376.
 */
int sid_flash_decode_fwd(const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* kv_indptr, const int32_t* kv_indices,
                         const int32_t* num_splits, int batch, int num_q_heads, int num_kv_heads,
                         int head_dim, int64_t num_slots, int max_splits, int fixed_split_size,
                         float sm_scale, float* part_o, float* part_lse, int part_batch,
                         int part_stride, void* o, void* stream);

/*
 * sid_flash_decode_fwd with every KV split cut into segments of at most
 * segment_size tokens (0: one segment per split), each computed by its own
 * workgroup; stage 2 merges all of a request's segments in token order.
 * Partial slot y of a request is segment y % sps of split y / sps, where
 * sps = ceil(chunk / min(segment_size, chunk)); grid_slots (<= part_stride)
 * slots are launched per request, so grid_slots must cover
 * max over requests of n_splits * sps (slots past a request's last segment
 * are empty and skipped). Same arguments and limits otherwise. The segment
 * size sets how many workgroups share a long split (the reference's grid is
 * one workgroup per head and split; here a workgroup reads all heads of its
 * tokens), and it is part of the reduction order: with a fixed split size
 * and a fixed segment size the result depends on the request alone. When
 * grid_slots == 1 the workspace is not touched. variant picks the stage-1
 * workgroup shape, which is part of the in-segment reduction order: 0 = 4
 * waves x 4 tokens per wave iteration (what sid_flash_decode_fwd uses), 1 =
 * 4 x 1 (full, HBM-bound grids), 2 = 8 x 2 (fewer workgroups than CUs), 3 =
 * 4 x 2 (in between); a fixed variant keeps the batch independence of fixed
 * splits. wg_order (may be NULL): int32 [batch * grid_slots], a permutation of
 * the grid's (request, slot) pairs packed as request << 12 | slot; the
 * stage-1 workgroup with linear id b + batch * y computes the pair at entry
 * b + batch * y. It changes which workgroup runs which segment, never the
 * result (a heaviest-first order balances ragged batches over the CUs);
 * entries outside the grid are skipped, so a map that is not a permutation
 * leaves partials unwritten (ABI 15). num_splits may be NULL here (not in
 * sid_flash_decode_fwd): each request's split count is then derived on the
 * device from its length, ceil(len / fixed_split_size) for fixed splits,
 * else min(ceil(len / 32), max_splits), the values the reference's policies
 * give (sid/kernels/decode_attention.py:65-85), with no host-side or
 * elementwise kernel to compute them (ABI 21).
 */
int sid_flash_decode_segments_fwd(const void* q, const void* k_cache, const void* v_cache,
                                  const int32_t* kv_indptr, const int32_t* kv_indices,
                                  const int32_t* num_splits, int batch, int num_q_heads,
                                  int num_kv_heads, int head_dim, int64_t num_slots,
                                  int max_splits, int fixed_split_size, int segment_size,
                                  int grid_slots, int variant, const int32_t* wg_order,
                                  float sm_scale, float* part_o, float* part_lse, int part_batch,
                                  int part_stride, void* o, void* stream);

/*
 * sid_flash_decode_segments_fwd with stage 1 run by `workers` workgroups that
 * each compute a share of the batch x grid_slots (request, slot) items in turn:
 * worker w takes the items at entries w, w + workers, w + 2 * workers, ... of
 * wg_order, which must then be a permutation of all of them (empty slots
 * included), packed as in sid_flash_decode_segments_fwd. Every item is computed
 * as the grid launch computes it, so the result is the same, bit for bit; the
 * caller deals the items so that the workers' token counts balance (ragged
 * batches, where the grid's workgroups cannot all be kept equally busy).
 * An entry with bit 30 set (SID_ORDER_EMPTY) is an item the caller knows to
 * hold no tokens; in each worker's sequence such entries must follow all of its
 * other entries. A worker marks them empty in one pass instead of visiting them
 * one by one (a flagged item that did hold tokens would be dropped from the
 * result). The grid launch ignores the flag.
 * workers == 0 is sid_flash_decode_segments_fwd. Ignored when grid_slots == 1.
 * Builds on sid_flash_decode_fwd (sid/csrc/flash_decode.cu:307-406): same
 * split geometry, partials and merge; the worker placement has no counterpart
 * in the reference (ABI 22).
 */
int sid_flash_decode_workers_fwd(const void* q, const void* k_cache, const void* v_cache,
                                 const int32_t* kv_indptr, const int32_t* kv_indices,
                                 const int32_t* num_splits, int batch, int num_q_heads,
                                 int num_kv_heads, int head_dim, int64_t num_slots,
                                 int max_splits, int fixed_split_size, int segment_size,
                                 int grid_slots, int variant, const int32_t* wg_order,
                                 float sm_scale, float* part_o, float* part_lse, int part_batch,
                                 int part_stride, void* o, int workers, void* stream);
#define SID_ORDER_EMPTY (1 << 30)

/*
 * No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): sid_flash_decode_segments_fwd without the part_o /
 * part_lse workspace. The split partials live in a static device array of
 * SID_DECODE_SCRATCH_BYTES per GPU (held until the process ends), laid out
 * as part_o [batch][HQ][grid_slots][D] fp32 followed (256-byte aligned) by
 * part_lse [batch][HQ][grid_slots]; a call that needs more returns an error
 * (SID_ERR_INVALID). Same kernels and bits as the workspace version. Nothing is
 * allocated and nothing needs clearing (stage 2 reads only what stage 1 wrote
 * in the same call). Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (different streams, or threads) race and must be
 * serialized by the caller. The first call on a device resolves the array's
 * device address (hipGetSymbolAddress) with that device current.
 */
#define SID_DECODE_SCRATCH_BYTES (32ll << 20)
int sid_flash_decode_segments_fwd_noalloc(const void* q, const void* k_cache,
                                          const void* v_cache, const int32_t* kv_indptr,
                                          const int32_t* kv_indices, const int32_t* num_splits,
                                          int batch, int num_q_heads, int num_kv_heads,
                                          int head_dim, int64_t num_slots, int max_splits,
                                          int fixed_split_size, int segment_size,
                                          int grid_slots, int variant, const int32_t* wg_order,
                                          float sm_scale, void* o,
                                          void* stream);

/* Size of that scratch array in bytes (SID_DECODE_SCRATCH_BYTES). */
int64_t sid_flash_decode_noalloc_scratch_bytes(void);

/*
 * Varlen causal attention over the paged pool (prefill, DVR verify). q, o:
 * bf16 [Text, HQ, D]; qo_indptr, kv_indptr int32 [B+1] (kv = prefix +
 * extend, all of it already in the pool); kv_indices int32. Query j of
 * request b sits at absolute position prefix_b + j and sees keys
 * 0 .. prefix_b + j. max_kv_len: an upper bound of every request's kv length
 * (sizes the split grid). Keys are reduced in 256-position splits anchored at
 * absolute position 0 and folded in split order, so a query's result depends
 * only on its absolute position and its sequence's keys (window-offset and
 * batch-slot invariant, bit for bit). workspace (optional, any alignment of
 * 16 bytes, sid_extend_attention_workspace_bytes(...) bytes) lets small
 * grids give each split its own workgroup; the result is bitwise the same
 * with or without it.
 * Replaces extend_attention_fwd, sid/kernels/extend_attention.py:115-144.
 */
int sid_extend_attention_fwd(const void* q, const void* k_cache, const void* v_cache,
                             const int32_t* qo_indptr, const int32_t* kv_indptr,
                             const int32_t* kv_indices, int batch, int64_t total_q,
                             int num_q_heads, int num_kv_heads, int head_dim, int64_t num_slots,
                             int max_extend_len, int max_kv_len, float sm_scale, void* workspace,
                             int64_t workspace_bytes, void* o, void* stream);

/* Workspace bytes sid_extend_attention_fwd uses for split fan-out; 0 = it does not fan out. */
int64_t sid_extend_attention_workspace_bytes(int batch, int64_t total_q, int num_q_heads,
                                             int num_kv_heads, int max_extend_len,
                                             int max_kv_len);

/*
 * out[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * w, fp32 math, bf16 I/O.
 * x, out: bf16 [rows, hidden]; w: bf16 [hidden]; hidden a multiple of 8,
 * at most 8192. out may alias x.
 * Replaces rmsnorm / qk_head_rmsnorm, sid/kernels/rmsnorm.py:45-55, 72-75.
 */
int sid_rmsnorm(const void* x, const void* w, void* out, int64_t rows, int hidden, float eps,
                void* stream);

/*
 * In place: residual += x (stored as bf16); x = rmsnorm(residual) where the
 * norm reads the fp32 sum before rounding. x, residual: bf16 [rows, hidden].
 * Replaces fused_add_rmsnorm, sid/kernels/rmsnorm.py:58-69 (kernel :27-42).
 */
int sid_fused_add_rmsnorm(void* x, void* residual, const void* w, int64_t rows, int hidden,
                          float eps, void* stream);

/*
 * sid_fused_add_rmsnorm with the x operand given as sid_linear_partials
 * output (nchunks chunk tiles of [rows, hidden]): x = bf16(fold(partials));
 * residual += x (stored as bf16); out = rmsnorm(residual). Bit-identical to
 * sid_linear followed by sid_fused_add_rmsnorm. Replaces the o/down
 * projection + fused_add_rmsnorm pair, sid/model/qwen3.py:80, 86, 104-108.
 */
int sid_fused_add_rmsnorm_partials(const float* partials, int nchunks, void* residual,
                                   const void* w, void* out, int64_t rows, int hidden, float eps,
                                   void* stream);

/*
 * NeoX rotate-half RoPE in place on q bf16 [T, HQ, D] and k bf16 [T, HKV, D]
 * at positions int64 [T], using cos_sin fp32 [max_positions, D] =
 * [cos(D/2) | sin(D/2)]. Tokens whose position is outside [0, max_positions)
 * are left unchanged. Replaces RotaryEmbedding.apply, sid/kernels/rope.py:50-61
 * (kernel :15-37).
 */
int sid_rope_apply(void* q, void* k, const int64_t* positions, const float* cos_sin,
                   int64_t num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                   int64_t max_positions, void* stream);

/*
 * y = x @ w^T (+ bias). x: bf16 [M, K] with row stride ldx (elements);
 * w: bf16 [N, K] contiguous (HF layout); bias: bf16 [N] or NULL; y: [M, N]
 * contiguous, bf16 when out_fp32 == 0, else fp32 holding the bf16-rounded
 * value (the reference's `linear(...).float()`). K must be a multiple of 256,
 * N a multiple of 64.
 * The reduction order of every output element is fixed and independent of M
 * (K in 256-wide chunks, each accumulated from zero in increasing k, chunk
 * sums added in increasing chunk order, then the bias, then one rounding),
 * so each row is bitwise identical whatever batch it is computed in.
 * Replaces F.linear / bi_linear / matmul_persistent at sid/model/qwen3.py:49,
 * 80, 84, 86, 114 and sid/kernels/matmul_persistent.py:82-113.
 */
int sid_linear(const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t m,
               int64_t n, int64_t k, int out_fp32, void* stream);

/*
 * Split-K form of sid_linear without bias: partials fp32 [K/256][M][N] gets
 * the sum of each 256-wide K chunk (accumulated exactly as in sid_linear).
 * Folding the chunks in increasing order and rounding to bf16 gives
 * sid_linear's result bit for bit; the *_partials consumers below do that.
 * Used for the small-M decode projections, whose N alone is too small to
 * fill the GPU. Same shape rules as sid_linear.
 */
int sid_linear_partials(const void* x, int64_t ldx, const void* w, float* partials, int64_t m,
                        int64_t n, int64_t k, void* stream);

/*
 * out[t, i] = silu(gate[t, i]) * up[t, i] with gate = gate_up[t, :I] and
 * up = gate_up[t, I:], each op rounded to bf16 like torch's
 * `F.silu(gate) * up`. gate_up: bf16 [T, 2I]; out bf16 [T, I].
 * Replaces sid/model/qwen3.py:84-85.
 */
int sid_silu_mul(const void* gate_up, void* out, int64_t num_tokens, int64_t inter, void* stream);

/* sid_silu_mul with gate_up given as sid_linear_partials output [nchunks][T][2I]. */
int sid_silu_mul_partials(const float* partials, int nchunks, void* out, int64_t num_tokens,
                          int64_t inter, void* stream);

/*
 * The gate_up projection and SwiGLU in one launch: out[t, j] =
 * bf16(bf16(silu(g)) * u) with g = row j and u = row I + j of
 * x @ w^T (x bf16 [M, K] contiguous, w bf16 [2I, K]), both in sid_linear's
 * reduction order and rounding. Bit-identical to sid_linear_partials followed
 * by sid_silu_mul_partials (and to sid_linear followed by sid_silu_mul).
 * K must be 1024; I a multiple of 8; x and w 16-byte aligned. out bf16 [M, I].
 * From M = 96 (with I a multiple of 64) it runs as the tiled prefill GEMM
 * with the SwiGLU applied in its epilogue; the [M, 2I] projection is never
 * written.
 * Replaces sid/model/qwen3.py:84-85 (gate_up = F.linear(...);
 * F.silu(gate) * up) for decode-sized batches and prefill.
 */
int sid_linear_silu_mul(const void* x, const void* w, void* out, int64_t m, int64_t k,
                        int64_t inter, void* stream);

/*
 * Fused QKV epilogue of Qwen3 attention (sid/model/qwen3.py:49-61): row t of
 * the projection is [q (HQ*D) | k (HKV*D) | v (HKV*D)], given either as bf16
 * qkv [T, (HQ+2*HKV)*D] or as sid_linear_partials output (exactly one of qkv
 * and partials non-NULL). q and k get the per-head RMSNorm (weights q_norm,
 * k_norm bf16 [D]) then NeoX RoPE at positions[t] (cos_sin as in
 * sid_rope_apply); q goes to q_out bf16 [T, HQ, D]; k and v are written to
 * k_cache / v_cache [S, HKV, D] at slots[t] (slots outside [0, S) skipped).
 * Bit-identical to split + qk_head_rmsnorm + rope + reshape_and_cache.
 * D must be 128.
 */
int sid_qkv_post(const void* qkv, const float* partials, int nchunks, int64_t num_tokens,
                 int num_q_heads, int num_kv_heads, int head_dim, const void* q_norm,
                 const void* k_norm, float eps, const int64_t* positions, const float* cos_sin,
                 int64_t max_positions, const int64_t* slots, void* q_out, void* k_cache,
                 void* v_cache, int64_t num_slots, void* stream);

/*
 * Decode-step chain: the projections of a Qwen3 layer with their neighbours
 * fused in, for decode-sized M (sid/model/qwen3.py:43-86 for one token per
 * request). Each output is bit-identical to the unfused sequence of the
 * entry points above (same reduction orders), so they are a speed choice.
 *
 * The weights of these entry points are in the fragment-packed order made by
 * sid_pack_decode_weight (same size as the [N, K] weight).
 *
 * sid_linear_residual: y = x w^T (x bf16 [M, K] with row stride ldx, w the
 * packed bf16 [N, K]), then r = residual + bf16(y) in fp32, residual = bf16(r) (bf16
 * [M, N], in place) and r32 = r (fp32 [M, N]). Replaces self.o_proj /
 * self.down_proj + fused_add_rmsnorm's residual half (sid/model/qwen3.py:80,
 * 86; sid/kernels/rmsnorm.py:27-42); r32 is the value that add-norm
 * normalises. N a multiple of 128; K in {1024, 2048, 3072, 4096}.
 */
int sid_linear_residual(const void* x, int64_t ldx, const void* w, void* residual, float* r32,
                        int64_t m, int64_t n, int64_t k, void* stream);

/*
 * sid_rmsnorm_linear_silu_mul: out = silu(g) * u (sid_linear_silu_mul's bits)
 * of x = bf16(rmsnorm(src) * norm_w), src fp32 [M, hidden] (src_fp32 != 0:
 * an r32 from sid_linear_residual) or bf16; w = [gate rows | up rows]
 * bf16 [2I, hidden], packed with gate_up = 1; out bf16 [M, I]. Replaces the rmsnorm half of
 * fused_add_rmsnorm + gate_up_proj + silu * up (sid/model/qwen3.py:84-85).
 * hidden in {512, 1024}; I a multiple of 24.
 */
int sid_rmsnorm_linear_silu_mul(const void* src, int src_fp32, const void* norm_w, float eps,
                                const void* w, void* out, int64_t m, int64_t hidden,
                                int64_t inter, void* stream);

/*
 * sid_rmsnorm_qkv_post: sid_qkv_post over the projection of
 * x = bf16(rmsnorm(src) * norm_w) by w_qkv bf16 [(HQ + 2 HKV) D, hidden]
 * (packed; src as above). Replaces the input rmsnorm / fused_add_rmsnorm + qkv_proj +
 * q/k-norm + RoPE + reshape_and_cache (sid/model/qwen3.py:49-61, 99-106).
 * hidden in {512, 1024}; D must be 128.
 */
int sid_rmsnorm_qkv_post(const void* src, int src_fp32, const void* norm_w, float eps,
                         const void* w_qkv, int64_t m, int64_t hidden, int num_q_heads,
                         int num_kv_heads, int head_dim, const void* q_norm, const void* k_norm,
                         const int64_t* positions, const float* cos_sin, int64_t max_positions,
                         const int64_t* slots, void* q_out, void* k_cache, void* v_cache,
                         int64_t num_slots, void* stream);

/*
 * sid_rmsnorm_f32: out = bf16(rmsnorm(x) * w) for fp32 rows x [rows, hidden]
 * (the final norm of the chain, sid/model/qwen3.py:111, on an r32); the bits
 * of sid_rmsnorm on the same values. hidden in {512, 1024, 2048}.
 */
int sid_rmsnorm_f32(const float* x, const void* w, void* out, int64_t rows, int hidden,
                    float eps, void* stream);

/*
 * sid_pack_decode_weight: packed = w (bf16 [N, K]) in fragment order: for
 * 16-row block b, 256-wide chunk c, k-step s < 8 and lane l < 64, the 8 bf16
 * at ((b * K / 256 + c) * 8 + s) * 512 + 8 l are row(b, l % 16), columns
 * 256 c + 32 s + 8 (l / 16) .. +7, with row(b, r) = 16 b + r, or, for a
 * gate_up weight (gate_up != 0, N = 2 I), gate row 8 b + r for r < 8 and up
 * row I + 8 b + r - 8. N a multiple of 16, K of 256. Run once at load time.
 */
int sid_pack_decode_weight(const void* w, void* packed, int64_t n, int64_t k, int gate_up,
                           void* stream);

/*
 * out[i] = table[idx[i]] for bf16 rows of row_elems elements (row_elems a
 * multiple of 8). Indices outside [0, table_rows) produce a zero row.
 * Used for the embedding lookup (sid/model/qwen3.py:93) and the sampled-row
 * gather (sid/model/qwen3.py:113).
 */
int sid_gather_rows(const void* table, const int64_t* idx, void* out, int64_t n,
                    int64_t row_elems, int64_t table_rows, void* stream);

/*
 * Per-row sampling over fp32 logits [rows, cols] (row stride ld), the
 * reference's sample(), sid/engine/sampler.py:32-69: temperature <= 0 gives the
 * greedy argmax (as sid_argmax_rows); otherwise p = softmax(logits / T), ranks
 * by (p descending, index ascending), rank r kept iff r < top_k (top_k <= 0:
 * no limit) and the mass of the ranks before it <= top_p (top_p >= 1: no
 * limit; mass summed exactly in units of 2^-48, each p rounded down), rank 0
 * always kept, token = argmax over kept columns of log(p + 1e-10) +
 * gumbel(seed, position, column) (the reference's int64 hash,
 * sampler.py:22-29; first index on ties). temperatures, top_ps fp32 [rows];
 * top_ks, seeds, positions int64 [rows]; out int64 [rows]. workspace:
 * sid_sample_workspace_bytes(rows, cols) bytes.
 */
int64_t sid_sample_workspace_bytes(int64_t rows, int64_t cols);
int sid_sample_rows(const float* logits, int64_t ld, const float* temperatures,
                    const int64_t* top_ks, const float* top_ps, const int64_t* seeds,
                    const int64_t* positions, int64_t rows, int64_t cols, void* workspace,
                    int64_t workspace_bytes, int64_t* out, void* stream);

/*
 * Greedy lm_head: out_idx[r] = argmax over columns of (x @ w^T + bias)[r, :],
 * the logits taken as sid_linear computes them (bf16-rounded, fp32 storage)
 * and compared with sid_argmax_rows's order. Fuses the lm_head projection
 * (sid/model/qwen3.py:114-115) with the greedy branch of sample()
 * (sid/engine/sampler.py:38) for an all-greedy batch. logits may be NULL (not
 * written) or fp32 [M, N]. Any M >= 1; K a multiple of 256. Up to 64 rows with
 * K == 1024 stream the weights once; otherwise the tiled GEMM keeps one
 * candidate per 128-column tile, so N <= 128 x 8 x (CU count) (1,048,576 on
 * MI355X). Workspace of sid_linear_argmax_workspace_bytes(M) bytes, 16-byte
 * aligned.
 */
int64_t sid_linear_argmax_workspace_bytes(int64_t m);
int sid_linear_argmax(const void* x, int64_t ldx, const void* w, const void* bias, float* logits,
                      int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                      int64_t* out_idx, void* stream);

/*
 * Native executor of one Qwen3 forward over an extend batch (prefill or DVR
 * verify): the kernel sequence of sid/model/qwen3.py:88-115 issued from C++
 * (embedding, per layer: qkv projection + q/k-norm + RoPE + cache write,
 * extend attention, o projection + residual add + RMSNorm, gate_up + SwiGLU,
 * down projection + residual add + RMSNorm; then the sampled rows' lm_head).
 * Results are bit-identical to issuing the same entry points one by one. It
 * has no counterpart of its own in the reference, whose forward is Python.
 * A projection with N <= 2048 output columns uses the split-K path up to
 * 4 * split_k_max_tokens tokens, N <= 4096 up to split_k_max_tokens, wider ones
 * below split_k_max_tokens (the results are the same either way). When the
 * layer's packed weights (sid_pack_decode_weight) are given and the batch has
 * at most chain_max_tokens tokens, each layer instead runs the decode-step
 * chain (sid_rmsnorm_qkv_post, extend attention, sid_linear_residual,
 * sid_rmsnorm_linear_silu_mul, sid_linear_residual): the same bits in five
 * launches. Outputs: logits fp32 [R, vocab] and/or tokens int64 [R]
 * (R = num_samples, or num_tokens without sample_indices): the greedy argmax,
 * or with b->temperatures the fused sampler's draw (sid_linear_sample: rows
 * without a top-k / top-p limit; needs hidden 1024 and R <= 4096, R <= 256
 * for the streaming grouping).
 */
typedef struct {
  const void* input_ln;
  const void* qkv;
  const void* q_norm;
  const void* k_norm;
  const void* o;
  const void* post_ln;
  const void* gate_up;
  const void* down;
  void* k_cache;
  void* v_cache;
  /* fragment-packed copies of qkv, o, gate_up (gate_up = 1) and down, or all NULL */
  const void* qkv_packed;
  const void* o_packed;
  const void* gate_up_packed;
  const void* down_packed;
} sid_qwen3_layer;

typedef struct {
  int num_layers;
  int hidden;
  int num_q_heads;
  int num_kv_heads;
  int head_dim;
  int intermediate;
  int vocab;
  float rms_eps;
  float sm_scale;
  int split_k_max_tokens;
  int chain_max_tokens; /* batches up to this size take the chain (packed weights given) */
  int64_t num_slots;
  int64_t max_positions;
  const float* cos_sin;
  const void* embed;
  const void* final_norm;
  const void* lm_head;
  const sid_qwen3_layer* layers;
} sid_qwen3_model;

typedef struct {
  int64_t num_tokens;
  int batch;
  int max_extend_len;
  int max_kv_len;  /* <= 0: num_kv_indices */
  int64_t num_kv_indices;
  const int64_t* input_ids;
  const int64_t* positions;
  const int64_t* out_slots;
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int64_t* sample_indices; /* NULL: every token row */
  int64_t num_samples;
  /* Sampled rows' draw parameters (sid_linear_sample), or NULL: greedy argmax */
  const float* temperatures;
  const int64_t* seeds;
  const int64_t* sample_positions;
  int sample_flags; /* sid_linear_sample's grouping flags (2: column tiles) */
} sid_extend_batch;

int64_t sid_qwen3_extend_workspace_bytes(const sid_qwen3_model* m, const sid_extend_batch* b);
int sid_qwen3_extend_forward(const sid_qwen3_model* m, const sid_extend_batch* b, void* workspace,
                             int64_t workspace_bytes, float* logits, int64_t* tokens,
                             void* stream);

/*
 * lm_head + sampler without the logits: out[r] = the token the sampler
 * (sid/engine/sampler.py:32-69) draws from logits x[r] w^T (bf16 x [M, K] with
 * row stride ldx, w [N, K], K = 1024, N a multiple of 16; 1 <= M <= 4096 with
 * the 128-column tiles, M <= 256 with the streaming waves):
 * temperatures[r] <= 0: argmax (first index, NaN first); else
 * argmax_c log(softmax(l / T)_c + 1e-10) + gumbel(seeds[r], positions[r], c)
 * with the reference's hash, i.e. sample() with top_k <= 0 and top_p >= 1
 * (rows with a top-k / top-p limit need sid_sample_rows over the logits).
 * The logits have the bits of sid_linear's fp32 output; they are written to
 * `logits` (fp32 [M, N]) when it is not NULL. Workspace:
 * sid_linear_sample_workspace_bytes(M) bytes (0 for an M out of range; about
 * 57 KB per row on 256 CUs), 16-byte aligned. Replaces the
 * logits epilogue of Qwen3Model.forward (sid/model/qwen3.py:113-115) plus
 * sample() for untruncated rows. The softmax sum is accumulated over groups of
 * columns: streaming waves (up to 64 rows) or 128-column tiles (more rows, or
 * logits requested); a row's token depends only on the row and the grouping,
 * so a caller that needs tokens independent of the batch size fixes the
 * grouping: flag 2 = column tiles, flag 4 = streaming waves (no logits).
 * flag 1 = recompute every column of every stochastic row exactly instead of
 * certifying the per-group candidates (a check: same tokens, much slower).
 */
int64_t sid_linear_sample_workspace_bytes(int64_t m);
int sid_linear_sample(const void* x, int64_t ldx, const void* w, int64_t m, int64_t n, int64_t k,
                      const float* temperatures, const int64_t* seeds, const int64_t* positions,
                      void* workspace, int64_t workspace_bytes, int64_t* out, float* logits,
                      int flags, void* stream);

/*
 * out[r] = argmax(logits[r, :]) with first-index tie-break; fp32 logits
 * [rows, cols] with row stride ld; out int64 [rows]. NaN compares greater
 * than every number (torch.argmax semantics). Replaces the greedy branch of
 * sample(), sid/engine/sampler.py:37.
 */
int sid_argmax_rows(const float* logits, int64_t ld, int64_t* out, int64_t rows, int64_t cols,
                    void* stream);

/*
 * Device-side decode batch construction over page tables. Request b sits on
 * row rows[b] of the int32 block table [num_rows, max_pages] (page ids; page p
 * holds pool slots p*page_size .. p*page_size + page_size - 1, page_size a
 * power of two) and has L_b = kv_indptr[b+1] - kv_indptr[b] positions, the
 * last one being decoded now into slot new_slots[b] (int64 [B], chosen by the
 * host allocator). Writes kv_indices[kv_indptr[b] + i] =
 * table[row][i / page_size] * page_size + i % page_size for i < L_b - 1, and
 * new_slots[b] for i = L_b - 1; when that position opens a page
 * ((L_b - 1) % page_size == 0), stores its page id into the table for later
 * steps. Rows outside the table, L_b <= 0 or L_b beyond max_pages pages are
 * skipped. Replaces the per-request host loop of build_decode_batch
 * (sid/engine/batch.py:120-133) over the reference's token table
 * (sid/engine/kv_cache.py:45-47), which is the page_size 1 case.
 */
int sid_build_paged_decode_indices(int32_t* block_tables, int64_t max_pages, int64_t num_rows,
                                   int page_size, const int64_t* rows, const int64_t* new_slots,
                                   const int32_t* kv_indptr, int32_t* kv_indices, int batch,
                                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SID_HIP_H_ */
