/* nc_hip.h: the C ABI of nanocompile_amd's HIP library (libnc_hip.so), gfx950.
 *
 * Kernel entry points keep the reference's generated-kernel calling
 * convention (codegen_c.py:5-10, 254, 282-283):
 *
 *     int32_t nc_name(void **p, const int64_t *s);
 *
 * p[0] is the (first) output, p[1..] the operands, all DEVICE pointers to
 * contiguous row-major arrays; s holds the sizes (the reference's s[] holds
 * its graph symbols seq and past, runtime.py:255). A call only enqueues work
 * on the library stream and returns 0, NC_BAD_ARGS (a shape or pointer the
 * launcher rejects) or NC_LAUNCH_FAILED. A kernel that finds bad input at run
 * time (the reference's loopir.Fail, loopir.py:280-285, used by gather with
 * code 1, fusion.py:722) records its code in a device word that nc_sync()
 * returns, which the Python runtime maps to KernelError as the reference's
 * runtime.py:298-318 does. nc_last_error() explains the last non-zero code.
 *
 * Dtypes: i8 = int8_t, i32 = int32_t, f32 = float, i64 = int64_t.
 */
#ifndef NC_HIP_H
#define NC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NC_OK 0
#define NC_FAIL_INDEX 1
#define NC_BAD_ARGS 2
#define NC_LAUNCH_FAILED 3
#define NC_FAIL_CAPACITY 4   /* a position read from the device ran past the cache */

/* -- runtime ------------------------------------------------------------------
 * Replaces the reference's library loading and executor binding
 * (runtime.py:62-83 pool loading, codegen_c.py:71-81 nc_bind_pool): one
 * device, one stream, instead of one thread pool. */

const char *nc_last_error(void);
int32_t nc_device_count(void);
/* Bind the library to a device and create its stream (runtime.py:200-203). */
int32_t nc_init(int32_t device);
int32_t nc_device_info(char *arch, int64_t arch_len, int64_t *compute_units, int64_t *lds_bytes,
                       int64_t *hbm_bytes, int64_t *clock_khz);
/* HIP runtime and driver versions: with the arch and CU count, the machine
 * key of the tuning cache (the reference keys on compiler, CPU and threads,
 * autotune.py:481-484). */
int32_t nc_runtime_version(int64_t *runtime, int64_t *driver);
/* A hash of the library's kernel sources and build flags: part of the tuning
 * cache's key, so winners measured on one build are not reused on another
 * (the reference keys its caches on source and flags, codegen_c.py:303-313). */
const char *nc_library_digest(void);

/* Device memory: the reference's one 64-byte-aligned arena (runtime.py:39,
 * 239-243) becomes one hipMalloc arena the Python runtime carves up. */
void *nc_malloc(int64_t bytes);
int32_t nc_free(void *ptr);
void *nc_host_malloc(int64_t bytes);       /* pinned host staging */
int32_t nc_host_free(void *ptr);
int32_t nc_memcpy_h2d(void *dst, const void *src, int64_t bytes);      /* waits */
int32_t nc_memcpy_d2h(void *dst, const void *src, int64_t bytes);      /* waits */
int32_t nc_memcpy_h2d_async(void *dst, const void *src, int64_t bytes);
int32_t nc_memcpy_d2h_async(void *dst, const void *src, int64_t bytes);
int32_t nc_memcpy_d2d(void *dst, const void *src, int64_t bytes);
/* height rows of width bytes, each side with its own pitch; kind 1 = host to
 * device, 2 = device to host; waits. The Runner path moves the rows of the
 * KV cache it does not hold on either side: the reference hands its cache
 * over as a view of one host buffer per call (models/qwen2.py:232-271,
 * 337-342), [layers, kv_heads, capacity, head_dim], whose (layer, head)
 * blocks are rows of a uniform pitch. */
int32_t nc_memcpy_rows(void *dst, int64_t dst_pitch, const void *src, int64_t src_pitch, int64_t width,
                       int64_t height, int32_t kind);

/* Wait for the stream; returns the first kernel failure code since the last
 * call (clearing it), NC_LAUNCH_FAILED, or 0 (runtime.py:298-299). */
int32_t nc_sync(void);
void *nc_stream_handle(void);
void *nc_error_word(void);

/* Events on the library stream: the reference times kernels with a C loop
 * around calls (autotune.py:89-122); here the GPU timestamps them. */
void *nc_event_create(void);
int32_t nc_event_record(void *event);
int32_t nc_event_elapsed_ms(void *start, void *stop, float *ms);
int32_t nc_event_destroy(void *event);

/* Graph capture of the library stream: a decode step's launches recorded
 * once and replayed (the reference's planned phase 7, docs/ROADMAP.md:209-228). */
int32_t nc_capture_begin(void);
int32_t nc_capture_end(void **graph_exec);
int32_t nc_graph_launch(void *graph_exec);
int32_t nc_graph_destroy(void *graph_exec);

/* -- int8 quantizers ---------------------------------------------------------- */

/* Per-row symmetric int8 weights (quantize.py:55-70, the reference's
 * quantize_int8, done on the host there).
 * p: [q i8[N,K], scales f32[N], w f32[N,K]];  s: [N, K] */
int32_t nc_quantize_rows_i8(void **p, const int64_t *s);

/* Per-token int8 activations: the reference's block quantizer
 * (quantize.py:102-124) with one block spanning the row.
 * p: [xq i8[M,K], xs f32[M], x f32[M,K]];  s: [M, K] */
int32_t nc_quantize_token_i8(void **p, const int64_t *s);

/* rms_norm (nn.py:34-38, one row kernel as fusion.py:631-650 makes it) fused
 * with the per-token quantizer.
 * p: [normed f32[M,K] or NULL, xq i8[M,K], xs f32[M], x f32[M,K], gamma f32[K]];
 * s: [M, K, eps as the bits of a float32] */
int32_t nc_rms_norm_quant(void **p, const int64_t *s);

/* Diagnostic: the device's float32 a / b, sqrt(|a|) and roundf(a), so tests can
 * hold them to IEEE correct rounding as the reference's C is (libm sqrtf and
 * '/', codegen_c.py:58, 141; roundf half away from zero, loopir.py:88-90).
 * p: [quotient f32[n], root f32[n], rounded f32[n], a f32[n], b f32[n]];  s: [n] */
int32_t nc_probe_fp32_ops(void **p, const int64_t *s);

/* -- int8 projections --------------------------------------------------------- */

/* matmul_i8_token: per-token int8 activations times per-row int8 weights,
 * int32 accumulation, fp32 epilogue y = (f32(acc) * xs[m]) * scales[n],
 * then + bias[n], then residual[m,n] + y. Extends the reference's int8
 * matmuls (ir.py:392-439, lowered at lower.py:400-417 and fused with bias,
 * residual and SwiGLU epilogues at fusion.py:677-711) with the per-token mode
 * the reference lacks.
 * p: [y f32[M,N], xq i8[M,K], xs f32[M], q i8[N,K], scales f32[N],
 *     bias f32[N] or NULL, residual f32[M,N] or NULL];
 * s: [M, N, K, schedule]. Schedules (the reference's schedule knobs,
 * schedules.py:96-110, become GPU launch shapes): 0 = the library's choice
 * (the GEMV below 16 tokens, else an MFMA tile chosen by shape);
 * 1..7 = the decode GEMV (lanes per row x waves per workgroup);
 * 16..24 = the MFMA GEMM on v_mfma_i32_16x16x64_i8 with LDS-staged tiles
 * (tile m x n, k stage, wave tile, register stages in flight), K a multiple of 16.
 * nc_schedule_info describes each. Every schedule computes the same bits. */
int32_t nc_matmul_i8_token(void **p, const int64_t *s);

/* A schedule's launch shape, for the tuner (no device call): out[0] = 0 for
 * the GEMV, then [lanes per row, waves, bytes per load]; out[0] = 1 for the
 * MFMA GEMM, then [tile m, tile n, k stage, wave m, wave n, register stages,
 * threads, LDS bytes with one weight matrix, LDS bytes with the SwiGLU pair's
 * two]. NC_BAD_ARGS for 0 or an unknown index. The
 * reference's schedule space is schedules.SPACES (schedules.py:96). */
int32_t nc_schedule_info(int32_t schedule, int64_t *out);

/* The raw int32 accumulators of matmul_i8_token, for bit-exact checking.
 * p: [acc i32[M,N], xq i8[M,K], q i8[N,K]];  s: [M, N, K, schedule] */
int32_t nc_matmul_i8_token_acc(void **p, const int64_t *s);

/* B independent matmul_i8_token problems in one launch, problem b reading its
 * own weights: a stream of decode projections over distinct weights (the
 * reference streams rotated weight copies for the same reason,
 * autotune.py:82-83, 181-182), measured as one kernel.
 * p: [y f32[B,M,N], xq i8[B,M,K], xs f32[B,M], q i8[B,N,K], scales f32[B,N]];
 * s: [B, M, N, K, schedule] */
int32_t nc_matmul_i8_token_stacked(void **p, const int64_t *s);

/* SwiGLU's gate and up projections sharing one pass over the activations
 * (fusion.py:677-711 shares their k loop), then h = silu(gate) * up
 * (nn.py:41-54) in the epilogue; each projection's epilogue as above.
 * p: [h f32[M,N], xq i8[M,K], xs f32[M], qg i8[N,K], sg f32[N], qu i8[N,K], su f32[N]];
 * s: [M, N, K, schedule] (K a multiple of 16, at most 8192; schedule 0, the
 * GEMV 7, or an MFMA tile 16..24) */
int32_t nc_matmul_i8_token_swiglu(void **p, const int64_t *s);

/* -- the reference's own int8 modes, bit for bit ------------------------------ */

/* matmul_i8: y = x @ (q * scales).T with f32 activations times int8 weights,
 * each dot summed in the reference's 32 interleaved chains then its tree
 * (lower.py:298-360, kernel at lower.py:400-417), then + bias, then
 * residual + y. The packed operand is q reordered chain-major once per weight
 * (nanocompile_amd.kernels.pack_chains) so the chains load coalesced.
 * p: [y f32[M,N], x f32[M,K], packed i8, q i8[N,K], scales f32[N],
 *     bias f32[N] or NULL, residual f32[M,N] or NULL];  s: [M, N, K] (K <= 16384) */
int32_t nc_matmul_i8(void **p, const int64_t *s);

/* rms_norm (nc_rms_norm_index_order, nn.py:34-38) of x's rows, then matmul_i8
 * (as nc_matmul_i8, lower.py:298-360) of the normalized rows, in one launch: every
 * workgroup normalizes its row the same way, so the result is bit for bit the two
 * calls'; it saves the norm's launch and its round trip through memory. At the
 * model's widths only (K 896 or 4864, x 16-byte aligned); y and residual must not
 * be x.
 * p: [y f32[M,N], x f32[M,K], packed i8, q i8[N,K], scales f32[N],
 *     bias f32[N] or NULL, residual f32[M,N] or NULL, gamma f32[K]];
 * s: [M, N, K, eps as float32 bits] */
int32_t nc_matmul_i8_normed(void **p, const int64_t *s);

/* The up projection with SwiGLU (nn.py:41-54, nc_silu_mul's operations) in its
 * epilogue: h = silu(gate) * matmul_i8(x, up), bit for bit the two calls'. At the
 * model's widths (K 896 or 4864, x 16-byte aligned; h not x).
 * p: [h f32[M,N], x f32[M,K], packed i8, q i8[N,K], scales f32[N], gate f32[M,N]];
 * s: [M, N, K] */
int32_t nc_matmul_i8_silu(void **p, const int64_t *s);

/* matmul_i8_vnni: per-block int8 activations (xq, xs, offset from
 * nc_quantize_blocks) times int8 weights, each block's byte dots in the
 * reference's Dp4 order with its +128 offset (lower.py:363-397), the block
 * sums scaled by xs and added in order, minus offset, times scales[n].
 * p: [y f32[M,N], xq i8[M,K], xs f32[M,K/block], offset f32[M], packed i8
 *     (pack_chains_vnni), q i8[N,K], scales f32[N], bias or NULL, residual or NULL];
 * s: [M, N, K, block] (block a power of two >= 32 dividing K) */
int32_t nc_matmul_i8_vnni(void **p, const int64_t *s);

/* matmul_i8_vnni of the up projection with SwiGLU in its epilogue, as
 * nc_matmul_i8_silu (K 896 or 4864, xq 16-byte aligned).
 * p: [h f32[M,N], xq i8[M,K], xs f32[M,K/block], offset f32[M], packed i8, q i8[N,K],
 *     scales f32[N], gate f32[M,N]];  s: [M, N, K, block] */
int32_t nc_matmul_i8_vnni_silu(void **p, const int64_t *s);

/* The block activation quantizer of matmul_i8_vnni (quantize.py:102-124):
 * per block of K, xs = max|x| / 127 (1 for an all-zero block), xq = round(x / xs),
 * offset = 128 * sum_b xs[b] * sum_{k in b} xq[k].
 * p: [xq i8[M,K], xs f32[M,K/block], offset f32[M], x f32[M,K]];  s: [M, K, block] */
int32_t nc_quantize_blocks(void **p, const int64_t *s);

/* rms_norm (nc_rms_norm_index_order, nn.py:34-38) of x's rows, then the block
 * quantizer (as nc_quantize_blocks, quantize.py:102-124, blocks of 32) of the
 * normalized rows, in one launch and one workgroup a row: bit for bit the two
 * calls', the norm's launch and its round trip through memory saved (int8-vnni's
 * norms feed nothing else).
 * p: [xq i8[M,K], xs f32[M,K/32], offset f32[M], x f32[M,K], gamma f32[K]];
 * s: [M, K, eps as float32 bits] (K a multiple of 64, at most 1024) */
int32_t nc_quantize_blocks_normed(void **p, const int64_t *s);

/* The reference's rms_norm in its own order (nn.py:34-38 as fusion.py:631-650
 * emits it: the row's sum of squares in index order), for the reference modes,
 * whose int8-vnni activations round after every norm and so need its bits.
 * p: [normed f32[M,K], x f32[M,K], gamma f32[K]];  s: [M, K, eps as float32 bits] */
int32_t nc_rms_norm_index_order(void **p, const int64_t *s);

/* The reference's attention in its own order (models/qwen2.py:143-147 with
 * nn.py:57-66 and the causal mask nn.py:123-135): each score a dot product in
 * order of d, times scale, plus the mask; exp(z - max); the sum in order of
 * position; p = e / sum; the context summed in order of position. One
 * workgroup a (query row, head); after nc_rope_append has rotated q and
 * appended the rows' keys and values. For the reference modes.
 * p: [ctx f32[M, heads*D], qkv f32[M, (heads+2kv)*D], kcache f32[kv, capacity, D],
 *     vcache f32[kv, capacity, D], pos i64[1] | NULL (past read on the device)];
 * s: [M, heads, kv, D, past, capacity (at most 16000), scale as float32 bits] */
int32_t nc_attention_index_order(void **p, const int64_t *s);

/* -- one decode token, fused ---------------------------------------------------- */

/* One projection of a single token with its activation prologue fused
 * (the reference's fused rms_norm row kernel and matmul epilogues,
 * fusion.py:631-711, for M = 1): kind 0 = rms_norm + per-token quantize +
 * bias (q, k, v); 1 = per-token quantize + residual added into out (o, down);
 * 2 = rms_norm + quantize + SwiGLU pair (gate, up). Same arithmetic, bit for
 * bit, as nc_rms_norm_quant followed by nc_matmul_i8_token(_swiglu).
 * p: [out f32[N] (holds the residual for kind 1), x f32[K], gamma f32[K] or NULL,
 *     q i8[N,K], scales f32[N], bias f32[N] or NULL, q2 i8[N,K] or NULL, scales2 f32[N] or NULL];
 * s: [N, K, kind, eps as float32 bits, schedule]; K in {896, 4864} (and the test model's 128, 256);
 * other widths take the unfused kernels. schedule 0 is the library's launch shape; 1..5 a row of
 * the width's table of (lanes a row, waves a workgroup, bytes a load), for the tuner: the
 * reference's schedule knobs (schedules.py:87-128) as GPU launch shapes, every one the same bits. */
int32_t nc_decode_projection(void **p, const int64_t *s);

/* A decode projection schedule, for the tuner (no device call): out = [lanes a row, waves a
 * workgroup, bytes a load]; NC_BAD_ARGS when it does not exist for width K and kind. */
int32_t nc_decode_schedule_info(int64_t K, int64_t kind, int64_t schedule, int64_t *out);

/* Attention of one new token (models/qwen2.py:113-155 at seq = 1) with RoPE of
 * its q and k heads and the cache append fused in: the same arithmetic, bit for
 * bit, as nc_rope_append followed by nc_attention (the 64-key chunked order
 * both share). One workgroup per (64-key chunk, KV head) attends all the
 * group's query heads to its chunk; a second launch combines the chunks.
 * p: [ctx f32[heads*D], qkv f32[(heads+2*kv)*D] (unrotated), kcache f32[kv,C,D],
 *     vcache f32[kv,C,D], inv_freq f32[D/2], pos i64[1] or NULL (read in place of s[3]),
 *     rope table f32[2,C,D/2] from nc_rope_table or NULL (then cos and sin are computed),
 *     work f32 (the chunk results: heads * ceil(keys / 64) * (D + 2) floats, keys = C
 *     with pos, else past + 1)];
 * s: [heads, kv, D, past, C, scale as float32 bits, work bytes] (D 16, 32 or 64, C <= 16384) */
int32_t nc_attention_decode(void **p, const int64_t *s);

/* nc_attention_decode without an allocation or a workspace argument: the same
 * kernels and the same bits, the chunk results kept in a 1 MiB device array
 * the library holds on each GPU until the process ends (its address looked up
 * by nc_init). No counterpart in the reference: it is for callers that cannot
 * call hipMalloc or pass a workspace (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation). Calls that overlap on one
 * GPU share that array and race; consecutive calls need no clearing.
 * p: [ctx f32[heads*D], qkv f32[(heads+2*kv)*D] (unrotated), kcache f32[kv,C,D],
 *     vcache f32[kv,C,D], inv_freq f32[D/2], pos i64[1] or NULL, rope table f32[2,C,D/2] or NULL];
 * s: [heads, kv, D, past, C, scale as float32 bits]; NC_BAD_ARGS when
 * heads * ceil(keys / 64) * (D + 2) floats (keys = C with pos, else past + 1)
 * exceed 1 MiB (the model's 14 heads of 64 fit every capacity up to 16384). */
int32_t nc_attention_decode_static(void **p, const int64_t *s);

/* RoPE's cos and sin for every position of a cache, computed once with the
 * kernels' own nc_cosf / nc_sinf of f32(position) * inv_freq[i] (the reference
 * builds the same angles as rope_tables, nn.py:78-94).
 * p: [table f32[2,C,D/2] (cos, then sin), inv_freq f32[D/2]];  s: [C, D] */
int32_t nc_rope_table(void **p, const int64_t *s);

/* -- fused groups around the projections (nn.py, models/qwen2.py) ------------ */

/* y = silu(g) * u elementwise: p = 0 <= g, e = exp(p ? -g : g),
 * sigmoid = (p ? 1 : e) / (e + 1), y = (g * sigmoid) * u (nn.py:41-54).
 * p: [y f32[n], g f32[n], u f32[n]];  s: [n] */
int32_t nc_silu_mul(void **p, const int64_t *s);

/* RoPE with the half-split pairing (nn.py:69-106) at positions past..past+seq-1.
 * p: [y f32[heads,seq,D], x f32[heads,seq,D], inv_freq f32[D/2]];  s: [heads, seq, D, past] */
int32_t nc_rope(void **p, const int64_t *s);

/* softmax(s + causal mask) row by row (nn.py:57-66 with nn.py:123-135, one
 * row kernel as fusion makes it); masked entries come out 0.
 * p: [y f32[heads,seq,past+seq], s f32[heads,seq,past+seq]];  s: [heads, seq, past] */
int32_t nc_softmax_causal(void **p, const int64_t *s);

/* Rotates the q and k heads of each qkv row by RoPE (q in place) and appends
 * k and v to the cache at positions past+i (models/qwen2.py:134-145: keys are
 * cached after rotation).
 * cos and sin come from the cache's table (nc_rope_table) when given: the same bits.
 * p: [qkv f32[M,(heads+2*kv)*D], kcache f32[kv,C,D], vcache f32[kv,C,D], inv_freq f32[D/2],
 *     pos i64[1] or NULL, rope table f32[2,C,D/2] or NULL];
 * s: [M, heads, kv, D, past, C] */
int32_t nc_rope_append(void **p, const int64_t *s);

/* A prompt's qkv projection with RoPE and the cache append in its epilogue
 * (models/qwen2.py:113-145, the projection then rotate-and-cache): the bits of
 * nc_matmul_i8_token (bias, no residual) followed by nc_rope_append with the
 * cache's table, in one launch on MFMA tiles one head wide.
 * p: [qkv f32[M,W] (out), xq i8[M,K], xs f32[M], q i8[W,K], scales f32[W], bias f32[W] or NULL,
 *     kcache f32[kv,C,D], vcache f32[kv,C,D], rope table f32[2,C,D/2], pos i64[1] or NULL];
 * s: [M, W, K, heads, kv, D, past, C, schedule] (W = (heads + 2*kv)*D, D 32 or 64, K a multiple
 *    of 16; schedule 0 the library's tile, or an MFMA tile 16..24 whose n is one head) */
int32_t nc_matmul_i8_token_rope(void **p, const int64_t *s);

/* Grouped-query attention of each new row over the cache, causal
 * (models/qwen2.py:113-155; query head h reads KV head h / (heads / kv), the
 * reference's repeat_kv as index arithmetic, nn.py:109-120). The softmax and
 * the context are computed in 64-key chunks combined afterwards, the order
 * nc_attention_decode shares, so prefill and decode agree bit for bit. One
 * workgroup per (64-key chunk, KV head, 4 query rows) attends the rows' query
 * heads of the group to its chunk; a second launch combines the chunks. The
 * reference materializes the [heads, M, keys] scores instead (README.md:317).
 * With xq and xs, ctx's per-token int8 (nc_quantize_token_i8's bits) is written
 * too, by the combine itself when a row's chunk results fit its LDS.
 * p: [ctx f32[M,heads*D], qkv (q rotated), kcache, vcache, pos i64[1] or NULL,
 *     work f32 (the chunk results: heads * ceil(keys / 64) * (D + 2) floats per query
 *     row, keys = C with pos, else past + M; fewer than M rows' worth takes the rows
 *     in slabs), xq i8[M,heads*D] or NULL, xs f32[M] or NULL];
 * s: [M, heads, kv, D, past, C, scale as float32 bits, work bytes, schedule] (D 16, 32 or 64;
 *    at most 16384 keys; schedule 0 the library's query rows a chunk workgroup, 1..4 the
 *    tuner's choices, nc_attention_schedule_info; every schedule the same bits) */
int32_t nc_attention(void **p, const int64_t *s);

/* A prefill attention schedule, for the tuner (no device call): out = [query rows a chunk
 * workgroup]; NC_BAD_ARGS outside 1..4. */
int32_t nc_attention_schedule_info(int64_t schedule, int64_t *out);

/* -- the model's ends ---------------------------------------------------------- */

/* Embedding gather (lower.py:420-444); an id outside 0..V-1 records failure
 * code 1 for nc_sync, as the reference's gather Fail does (fusion.py:722).
 * p: [x f32[M,H], table f32[V,H], ids i64[M]];  s: [M, H, V] */
int32_t nc_embed(void **p, const int64_t *s);

/* The LM head's packed table: blocks of 64 rows, 4 consecutive k per row
 * together (the reference's pack, schedule.py:362-395).
 * p: [packed f32[ceil(V/64)*64, H], table f32[V,H]];  s: [V, H] */
int32_t nc_pack_rows64(void **p, const int64_t *s);

/* logits = x @ table.T with each row summed in k order, multiply then add
 * (the reference's float32 matmul kernel, lower.py:255-269), and best[m] the
 * 64-bit argmax key of row m (first index of the maximum). With gamma, x is
 * rms-normed first (eps = s[3] as float32 bits). With bias, + bias[n] after the
 * sum, and with residual, residual + that: the reference's float32 linear
 * (nn.py:24-31) and residual add, so the same kernel is the float32 model's
 * projections. With s[4] = 1 the argmax is left as one key per workgroup
 * (of 64 rows), best u64[M, G] with G = ceil(V/64), for nc_argmax_index or
 * nc_decode_advance to reduce (no atomics, nothing to clear); with s[4] = 0,
 * best u64[M] receives atomic maxima and must be cleared first.
 * p: [logits f32[M,V] or NULL, best or NULL, x f32[M,H], packed table,
 *     gamma f32[H] or NULL, bias f32[V] or NULL, residual f32[M,V] or NULL];
 * s: [M, V, H, eps bits, key per workgroup 0 or 1] */
int32_t nc_lm_head(void **p, const int64_t *s);

/* p: [best u64[n]];  s: [n]  (zeroes the argmax keys before nc_lm_head) */
int32_t nc_argmax_clear(void **p, const int64_t *s);

/* Argmax keys to token ids: one key per row (G = 0), or each row's G
 * per-workgroup keys from nc_lm_head with s[4] = 1, reduced.
 * p: [index i64[n], best u64[n] or u64[n,G]];  s: [n, G] */
int32_t nc_argmax_index(void **p, const int64_t *s);

/* Greedy decoding's bookkeeping on the device (models/qwen2.py:362-367 does it
 * on the host): token = argmax of the step just run; tokens[pos + 1] = token;
 * ids[0] = token; pos += 1; the argmax key cleared. A captured decode step
 * ends with it, so steps chain with no host round trip. Records
 * NC_FAIL_CAPACITY when pos + 1 reaches the capacity. With x, the token's
 * embedding row is gathered into x as well (nc_embed's gather and Fail code 1),
 * so the next step needs no separate embedding launch.
 * With G > 0, best holds nc_lm_head's G per-workgroup keys, reduced here.
 * p: [ids i64[1], tokens i64[capacity], best u64[1] or u64[G], pos i64[1], x f32[H] or NULL,
 *     table f32[V,H] or NULL];  s: [capacity, H, V, G] (H, V read only with x)
 * nc_rope_append and nc_attention take pos as an optional p[4], read on the
 * device in place of s[4] (past). */
int32_t nc_decode_advance(void **p, const int64_t *s);

#ifdef __cplusplus
}
#endif

#endif /* NC_HIP_H */
