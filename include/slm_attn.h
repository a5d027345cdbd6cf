/*
 * slm_attn -- MI355X (gfx950) attention hot path of static-lm behind a C ABI.
 *
 * Covers, on one GPU:
 *   - RoPE on q and k with host-computed cos/sin tables
 *       (transformer.rs:103-133 tables, :178-194 apply_rope_cached);
 *   - KV-cache append into the arena layout [layer][K|V][max_seq_len][kv_dim]
 *       f32 (transformer.rs:323-338, 413-428, 530-578; arena.rs:95-113);
 *   - causal multi-head / grouped-query attention for one decode position
 *       (causal_multi_head_attention_jit, transformer.rs:273-321) and for a
 *       batched prefill (the per-row loop of transformer.rs:563-593).
 *
 * (transformer.rs = src/model/transformer.rs, arena.rs = src/memory/arena.rs
 * of static-lm.)
 *
 * Conventions
 *   - Every function returns SLM_OK (0) or a negative SLM_ERR_* code; nothing
 *     aborts.  slm_attn_last_error() gives the message.  Each code mirrors one
 *     reference assert!, so a Rust wrapper can panic!() on nonzero to keep the
 *     reference behaviour.
 *   - A context is not thread-safe (it mirrors `&mut AlignedArena`); separate
 *     contexts are independent.  Each context owns one HIP stream (default
 *     priority, blocking: ordered with the legacy default stream) unless
 *     slm_attn_set_stream() hands it another.
 *   - Host-pointer entry points are synchronous and borrow their buffers for
 *     the call only.  *_dev entry points take device pointers, are enqueued on
 *     the context stream and return without waiting.
 *   - Device memory (KV region, RoPE tables, split-K partials) is owned by
 *     the context.
 *   - The reference's `att` scratch (H * max_seq_len floats, written and never
 *     read after the call) is not exposed: the kernels keep scores on chip.
 */
#ifndef SLM_ATTN_H
#define SLM_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SLM_OK 0
/* A LayerWorkspace::allocate assert failed (transformer.rs:81-101), or
 * num_layers/max_seq_len/rope_theta is not positive. */
#define SLM_ERR_CONFIG (-1)
/* pos >= max_seq_len ("sequence position out of bounds", transformer.rs:404-407). */
#define SLM_ERR_POS (-2)
/* n == 0 or start + n > max_seq_len (transformer.rs:501-502). */
#define SLM_ERR_BATCH (-3)
/* layer index outside 0..num_layers (the layer-count assert, transformer.rs:761-766). */
#define SLM_ERR_LAYER (-4)
/* out overlaps q, k, v or the KV region (attention_slices, arena.rs:272-280),
 * or an input of an appending call (decode, prefill, KV append) overlaps the
 * KV region: k and v are staging rows, not cache rows. */
#define SLM_ERR_ALIAS (-5)
/* NULL pointer, which not in {0,1}, or a row range outside the cache
 * (ArenaSlice::subslice bounds, arena.rs:27-36). */
#define SLM_ERR_ARG (-6)
/* The HIP runtime reported an error (message in slm_attn_last_error). */
#define SLM_ERR_HIP (-7)
/* head_dim outside the compiled set {16, 32, 48, 64, 96, 128, 256}. */
#define SLM_ERR_UNSUPPORTED (-8)
/* No gfx950 device, or the library's device code cannot run on it. */
#define SLM_ERR_DEVICE (-9)
/* The call cannot be recorded into a graph (it synchronizes, copies host
 * memory or would allocate) and the context's stream is being captured; or a
 * capture call out of order (slm_attn_capture_begin). */
#define SLM_ERR_CAPTURE (-23)

/* TransformerConfig fields that attention uses (transformer.rs:8-33) plus
 * the layer count and RoPE base.  The reference hard-codes the base to
 * 10000.0 (transformer.rs:128); 10000.0f reproduces it. */
typedef struct slm_attn_config {
    int32_t dim;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t max_seq_len;
    int32_t num_layers;
    float rope_theta;
} slm_attn_config;

typedef struct slm_attn_ctx slm_attn_ctx;

/* Validates the config like LayerWorkspace::allocate (transformer.rs:81-101),
 * computes the RoPE tables on the host exactly as transformer.rs:124-133 and
 * uploads them, and allocates the device KV region [L][2][msl][kv_dim] f32,
 * zeroed like AlignedArena::with_capacity (arena.rs:54-75).
 * Replaces TransformerModel::new's KV and table set-up (transformer.rs:714-743). */
int slm_attn_create(const slm_attn_config* cfg, slm_attn_ctx** out);

/* Frees everything the context owns (AlignedArena's Drop, arena.rs:296-303). */
void slm_attn_destroy(slm_attn_ctx* ctx);

/* Message for the last failed call on ctx (or on this thread, for ctx NULL). */
const char* slm_attn_last_error(const slm_attn_ctx* ctx);

/* ---- whole attention block ------------------------------------------------
 * Decode, transformer.rs:413-443: K row `pos` <- rope(k, pos), V row `pos`
 * <- v, q rotated, then causal attention of the rotated q over cache rows
 * 0..=pos; out[dim] receives the head outputs (the `xb` the Wo GEMV reads).
 * q: [dim], k, v: [kv_dim], out: [dim].  Host pointers, synchronous. */
int slm_attn_decode(slm_attn_ctx* ctx, int32_t layer, int32_t pos,
                    const float* q, const float* k, const float* v, float* out);

/* Prefill, transformer.rs:530-593: rows b < n sit at positions start + b;
 * K/V rows start..start+n-1 are appended (K rotated) and row b attends to
 * cache rows 0..=start+b.  start > 0 continues an earlier prefill.
 * q: [n][dim], k, v: [n][kv_dim], out: [n][dim].  Host pointers, synchronous. */
int slm_attn_prefill(slm_attn_ctx* ctx, int32_t layer, int32_t start,
                     int32_t n, const float* q, const float* k, const float* v,
                     float* out);

/* Same as slm_attn_decode / slm_attn_prefill on device pointers, enqueued on
 * the context stream. */
int slm_attn_decode_dev(slm_attn_ctx* ctx, int32_t layer, int32_t pos,
                        const float* q, const float* k, const float* v,
                        float* out);
int slm_attn_prefill_dev(slm_attn_ctx* ctx, int32_t layer, int32_t start,
                         int32_t n, const float* q, const float* k,
                         const float* v, float* out);

/* ---- the reference's separate steps, on device pointers ------------------
 * apply_rope_cached (transformer.rs:178-194) on n rows of row_len floats
 * (row_len a multiple of head_dim) at positions pos0..pos0+n-1, in place. */
int slm_rope_apply_dev(slm_attn_ctx* ctx, float* x, int32_t n, int32_t row_len,
                       int32_t pos0);

/* KV append: K rows pos0..pos0+n-1 of `layer` <- rope(k rows), V rows <- v
 * rows (transformer.rs:413-417 + 425-428 for n = 1; 545-561 + 575-578 for a
 * batch).  Bit-identical to the reference's f32 arithmetic. */
int slm_kv_append_dev(slm_attn_ctx* ctx, int32_t layer, int32_t pos0,
                      int32_t n, const float* k, const float* v);

/* causal_multi_head_attention_jit (transformer.rs:275-321) for an already
 * rotated q[dim] over cache rows 0..=pos of `layer`; writes out[dim]. */
int slm_attn_attend_dev(slm_attn_ctx* ctx, int32_t layer, int32_t pos,
                        const float* q_rot, float* out);

/* The per-row attention loop of transformer.rs:563-593 without the RoPE and
 * append steps: rotated q rows b < n attend to cache rows 0..=start+b. */
int slm_attn_attend_batch_dev(slm_attn_ctx* ctx, int32_t layer, int32_t start,
                              int32_t n, const float* q_rot, float* out);

/* ---- stream control ------------------------------------------------------- */
/* Use `stream` (a hipStream_t) for all later device work; NULL restores the
 * context's own stream. */
int slm_attn_set_stream(slm_attn_ctx* ctx, void* stream);
void* slm_attn_get_stream(const slm_attn_ctx* ctx);
/* Wait for all work enqueued on the context stream. */
int slm_attn_sync(slm_attn_ctx* ctx);

/* ---- HIP graphs ------------------------------------------------------------
 * No counterpart in the reference (its calls run on CPU threads).  For callers
 * that replay a fixed sequence of device-pointer calls (a serving loop, a
 * benchmark pass): between slm_attn_capture_begin and slm_attn_capture_end the
 * context's stream is captured (HIP stream capture, this thread only), so the
 * device-pointer entry points record their kernels instead of running them;
 * slm_attn_graph_launch replays the recording on the context's stream with one
 * host call.  A replay repeats the recorded arguments (positions, pointers):
 * the caller changes inputs in the device buffers between replays.  While
 * capturing, calls that synchronize, copy host memory, change the stream,
 * time kernels or would grow a workspace return SLM_ERR_CAPTURE and record
 * nothing (make one uncaptured call first to size workspaces).  Captured
 * launches carry no memset nodes.  Other work on the same stream during the
 * capture (from other libraries) is recorded too.  Destroy a graph only after
 * its replays have finished (slm_attn_sync), and before its context: the
 * recording holds the context's device buffers. */
typedef struct slm_attn_graph slm_attn_graph;
int slm_attn_capture_begin(slm_attn_ctx* ctx);
int slm_attn_capture_end(slm_attn_ctx* ctx, slm_attn_graph** out);
int slm_attn_graph_launch(slm_attn_ctx* ctx, const slm_attn_graph* graph);
void slm_attn_graph_destroy(slm_attn_graph* graph);

/* ---- raw KV cache access (pre-fill, snapshot/restore, bit-exact checks) ---
 * which: 0 = K, 1 = V.  Rows pos0..pos0+n-1, each kv_dim floats.  Host
 * buffers, synchronous. */
int slm_kv_write(slm_attn_ctx* ctx, int32_t layer, int32_t which, int32_t pos0,
                 int32_t n, const float* rows);
int slm_kv_read(slm_attn_ctx* ctx, int32_t layer, int32_t which, int32_t pos0,
                int32_t n, float* rows);
/* Same as slm_kv_write from a device buffer, enqueued on the context stream:
 * the path for a producer (e.g. a device-side Wk/Wv GEMV) that writes rows
 * the way the reference's GEMV writes them straight into the cache
 * (transformer.rs:416-417). */
int slm_kv_write_dev(slm_attn_ctx* ctx, int32_t layer, int32_t which,
                     int32_t pos0, int32_t n, const float* rows);

/* Float offset of row `pos` of K/V of `layer` from the region base:
 * ((2*layer + which) * max_seq_len + pos) * kv_dim -- the arena offsets of
 * LayerKvCache::allocate in layer order (transformer.rs:724-726) relative to
 * kv_caches[0].k_cache.offset.  Returns (size_t)-1 for bad arguments. */
size_t slm_kv_offset(const slm_attn_ctx* ctx, int32_t layer, int32_t which,
                     int32_t pos);

/* Device address of the KV region base, for producers that write final
 * (already rotated) rows in place and then call slm_attn_attend_dev /
 * slm_attn_attend_batch_dev.  The appending calls (decode, prefill, KV
 * append) refuse inputs that point into this region (SLM_ERR_ALIAS). */
float* slm_kv_device_ptr(const slm_attn_ctx* ctx);

/* Copy the device RoPE tables [max_seq_len][head_dim/2] back to the host. */
int slm_rope_tables_read(slm_attn_ctx* ctx, float* cos_out, float* sin_out);

/* ---- kernel timing -------------------------------------------------------
 * While enabled, every launch is timed with HIP events on the context
 * stream, and slm_attn_profile_read() returns, per kernel kind, the number
 * of launches and their summed duration in ms (it synchronizes the stream).
 * The decode and merge launches stamp their events at the kernel's own start
 * and end (as a kernel trace measures); other kinds are bracketed by events
 * recorded around the launch, which adds its dispatch (~2 us).
 * Reading resets the counters. */
enum {
    SLM_K_APPEND = 0,  /* rope(k) + KV append of a prefill batch */
    SLM_K_DECODE = 1,  /* decode: in-kernel KV append + split-K attention */
    SLM_K_COMBINE = 2, /* merge of the decode split partials */
    SLM_K_PREFILL = 3, /* causal prefill attention */
    SLM_K_ROPE = 4,    /* standalone rope */
    SLM_K_QUANT = 5,   /* Q8_0 activation quantization (slm_quant.h) */
    SLM_K_GEMM = 6,    /* Q4_0 x Q8_0 GEMV / GEMM (slm_quant.h) */
    SLM_K_NORM = 7,    /* RMSNorm / L2 norm (slm_layer.h) */
    SLM_K_ELEM = 8,    /* SwiGLU, residual add, embedding rows, argmax (slm_layer.h) */
    SLM_K_COUNT = 9
};
typedef struct slm_kernel_stat {
    int64_t launches;
    double total_ms;
} slm_kernel_stat;
int slm_attn_profile(slm_attn_ctx* ctx, int32_t enable);
int slm_attn_profile_read(slm_attn_ctx* ctx, slm_kernel_stat* out /* [SLM_K_COUNT] */);

/* Split-K layout the decode kernel uses at a given sequence length: positions
 * are cut into tiles of *tile rows and split s of *n_splits reads tiles s,
 * s + n_splits, s + 2*n_splits, ...  The tile length depends on the length too
 * for head_dim 16-96 (shorter tiles for short sequences).  A pure function of
 * seq_len, the config and the device's CU count, so results reproduce run to
 * run on a device. */
int slm_attn_decode_splits(const slm_attn_ctx* ctx, int32_t seq_len,
                           int32_t* n_splits, int32_t* tile);

/* The kernel a causal prefill of n rows from row start runs (slm_attn_prefill,
 * slm_attn_prefill_dev and the blocks built on them).  Like the decode split
 * layout, a pure function of start, n, the config and the device's CU count;
 * no counterpart in the reference, which has one scalar path: it is for tests
 * and benchmarks that need to know which kernel ran.  Heads per workgroup are
 * query heads of one KV head; query blocks are 16 rows; "paired" workgroups
 * take blocks i and n_blocks-1-i, so every workgroup has the same causal
 * work.  SLM_ERR_BATCH as slm_attn_prefill for an empty or out-of-range
 * batch. */
enum {
    SLM_PF_FOUR_HEADS = 0,        /* four heads, one block (kv_mul % 4 == 0) */
    SLM_PF_THREE_HEADS = 1,       /* three heads, one block (kv_mul % 3 == 0) */
    SLM_PF_TWO_HEADS = 2,         /* two heads, two blocks (kv_mul even) */
    SLM_PF_ONE_HEAD = 3,          /* one head, four blocks */
    SLM_PF_KEY_SPLIT = 4,         /* one head, one block, key tiles over four waves (hd <= 64) */
    SLM_PF_PAIRED_FOUR_HEADS = 5, /* four heads, paired blocks (hd <= 96) */
    SLM_PF_DMA = 6,               /* hd 128: four heads, two blocks, tiles staged by DMA */
    SLM_PF_DMA_PAIRED = 7,        /* hd 128: the same with paired blocks */
    SLM_PF_PAIRED_TWO_HEADS = 8,  /* hd 128: two heads, paired blocks, two key splits */
    SLM_PF_PAIRED_ONE_HEAD = 9    /* hd 128: one head, paired blocks, four key splits */
};
int slm_attn_prefill_kernel(const slm_attn_ctx* ctx, int32_t start, int32_t n,
                            int32_t* kernel);

/* Library version string. */
const char* slm_attn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SLM_ATTN_H */
