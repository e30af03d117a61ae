/*
 * oscar_hip.h -- C ABI of the MI355X (gfx950) OSCAR INT2 KV-cache hot path.
 *
 * Every entry point replaces one Python entry point of the reference plugin
 * (jpl123123/Oscar_new, package oscar_ascend, file kernels.py) and keeps its
 * argument meaning. Conventions:
 *   - device pointers are plain addresses; bf16 data is passed as 16-bit words;
 *   - strides are in ELEMENTS of the pointed-to type;
 *   - `stream` is a hipStream_t (NULL = default stream); launches are asynchronous,
 *     nothing synchronizes the host and nothing is read back to it;
 *   - no entry point allocates device memory (callers own every buffer), so all of
 *     them can be captured in a HIP graph;
 *   - return value: 0 on success, a negative OSCAR_E* code for an argument error
 *     detected on the host (nothing launched), or a positive hipError_t from the launch.
 * Device-side metadata (counts, task tables, block tables, slots) is trusted for
 * semantics but every history/window/table access is bounds-checked against the sizes
 * passed here; out-of-range entries are skipped, never dereferenced.
 */
#ifndef OSCAR_HIP_H_
#define OSCAR_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OSCAR_ABI_VERSION 1

enum oscar_status {
  OSCAR_OK = 0,
  OSCAR_E_NULL = -1,        /* a required pointer is NULL */
  OSCAR_E_SHAPE = -2,       /* sizes/strides inconsistent or unsupported */
  OSCAR_E_LAYOUT = -3,      /* cache geometry invalid */
  OSCAR_E_ALIGN = -4,       /* pointer or stride alignment not supported */
  OSCAR_E_UNSUPPORTED = -5, /* valid request outside this build's coverage */
  OSCAR_E_SCRATCH = -6      /* request larger than the fixed scratch of a no-alloc entry */
};

/* Cache geometry (reference: oscar_ascend/layout.py:9-44, config.py:45-63). */
typedef struct oscar_layout {
  int32_t head_dim;              /* D; must be 256 */
  int32_t kv_heads;              /* H */
  int32_t physical_block_tokens; /* Bp, tokens per physical page */
  int32_t kernel_block_tokens;   /* BK, tokens per block-table entry (power of two) */
  int32_t slot_bytes;            /* 160 */
  int32_t vector_bytes;          /* 68 */
  int32_t sink_tokens;           /* S */
  int32_t recent_tokens;         /* R */
  int32_t ring_tokens;           /* C = R + speculative + 1 */
  int32_t reserved;              /* 0 */
  int64_t stripe_page_bytes;     /* Bp * H * D * 2 */
} oscar_layout;

/* Clip configuration (reference: config.py:14-19; kernels.py:69-101). */
enum oscar_clip_mode {
  OSCAR_CLIP_PERCENTILE = 0, /* torch.quantile(|x|, ratio) threshold; ratio 0 = off */
  OSCAR_CLIP_FACTOR = 1,     /* max|x| * factor */
  OSCAR_CLIP_SEARCH = 2      /* argmin-MSE over factors 0.6 + 0.4*i/7, i = 0..7 */
};

typedef struct oscar_clip {
  int32_t mode;
  float k_ratio, v_ratio;   /* percentile mode */
  float k_factor, v_factor; /* factor mode */
} oscar_clip;

int oscar_abi_version(void);
const char* oscar_status_string(int status);

/*
 * rotate -- replaces kernels.py:51-66 `rotate(x, rotation)`.
 * out[t, h, :] = bf16( x[t, h, :] @ R ), fp32 accumulation on bf16 MFMA.
 * x: bf16 [n, h, d] with strides (x_s0, x_s1, x_s2); R: bf16 [d, d] with strides
 * (r_s0, r_s1) -- a transposed view (r_s0 = 1) is allowed; out: contiguous bf16 [n, h, d].
 * d must be 256.
 */
int oscar_rotate(const void* x, int64_t n, int64_t h, int64_t d, int64_t x_s0, int64_t x_s1,
                 int64_t x_s2, const void* rotation, int64_t r_s0, int64_t r_s1, void* out,
                 void* stream);

/*
 * store_int2 -- replaces kernels.py:175-202 `store_int2(key_rot, value_rot, history,
 * slots, counts, layout)`.
 * For every token t < counts[1] with slots[t] >= 0 and head h: clip, INT2-quantize and
 * pack key_rot[t, h] to bytes [0, 68) and value_rot[t, h] to bytes [68, 136) of the
 * 160-byte slot at layout slot_offset(slots[t], h). Bytes 136..159 are never written.
 * key_rot/value_rot: contiguous bf16 [n, H, 256]; history: K stripe bytes.
 * n * H must be below 2^31 (OSCAR_E_SHAPE otherwise).
 */
int oscar_store_int2(const void* key_rot, const void* value_rot, int64_t n, void* history,
                     int64_t history_bytes, const int64_t* slots, const int32_t* counts,
                     const oscar_layout* layout, const oscar_clip* clip, void* stream);

/*
 * rotate_store_int2 -- replaces the reference's `store_int2(rotate(key, Rk), rotate(value,
 * Rv), ...)` sequence (backend.py:171-173; kernels.py:51-66 and 175-202) with one launch:
 * the same cache bytes as oscar_rotate of K and V followed by oscar_store_int2, without the
 * rotated rows going through HBM. key/value: bf16 [n][kv_heads][256], row (token, head) at
 * token * s0 + head * s1 elements (s0, s1 multiples of 8; rows contiguous, 16-byte aligned).
 * rk_t / rv_t: R_k^T and R_v^T, contiguous bf16 [256][256]. No reference counterpart as one
 * call.
 */
int oscar_rotate_store_int2(const void* key, int64_t k_s0, int64_t k_s1, const void* value,
                            int64_t v_s0, int64_t v_s1, int64_t n, const void* rk_t,
                            const void* rv_t, void* history, int64_t history_bytes,
                            const int64_t* slots, const int32_t* counts,
                            const oscar_layout* layout, const oscar_clip* clip, void* stream);

/*
 * prepare_tasks -- replaces kernels.py:262-287 `prepare_tasks(qstarts, counts, tasks,
 * task_count, max_reqs, query_tile, num_reqs, source_table, table, copy_columns)`.
 * Writes tasks[i] = (req, q_offset) for every query tile of every request < counts[0]
 * (requests in order, tiles of query_tile tokens clipped to counts[1]) and
 * task_count[0] = number of tasks. `programs` is the reference grid size
 * (num_reqs, or max_reqs when num_reqs is None). If source_table != NULL the first
 * copy_columns columns of each live request row are copied into table.
 * task_capacity bounds the rows written to tasks.
 */
int oscar_prepare_tasks(const int32_t* qstarts, const int32_t* counts, int32_t* tasks,
                        int32_t* task_count, int64_t task_capacity, int64_t max_reqs,
                        int32_t query_tile, int64_t programs, const int32_t* source_table,
                        int64_t source_stride, int32_t* table, int64_t table_stride,
                        int64_t copy_columns, void* stream);

/*
 * attention_partials -- replaces kernels.py:439-482 `attention_partials(query, key,
 * value, history, window, meta, layout, scale, splits, raw)`.
 * Grid (programs, H, splits): program i serves task i if i < task_count[0]; `tasks` must
 * hold `programs` rows (prepare_tasks' task_capacity >= programs), all of which are read.
 * raw == 0: INT2 history positions [min(S, prefix), max(sink_len, prefix - R)) read from
 *           `history` through `block_tables` (query must be the ROTATED query);
 * raw != 0: BF16 sink/ring window positions plus the causal current tokens (key/value).
 * partials: fp32 [n, hq, splits, 256]; lse: fp32 [n, hq, splits] (natural log).
 * Live rows of an empty split get 0 / -inf; rows of inactive programs are not written.
 * Split boundaries follow kernels.py:368-370 with block_n tokens per tile.
 * split_tokens (history branch only; 0 = the reference rule above): a request with L history
 * tokens uses min(splits, max(1, ceil(L / split_tokens))) splits, its ranges following the
 * same rule with that count except that inner boundaries move down to the 64-token grid of
 * absolute positions; the split slots above it get lse -inf and no partial row (no
 * reference counterpart: for ragged batches, whose long requests would otherwise hold the
 * whole launch). raw != 0 requires split_tokens == 0.
 * queue_counters: NULL, or two int32 counters, zero before the first call, that a launch
 * leaves zero again (no reference counterpart). With them, a history launch of 17-32 rows
 * per task with split_tokens > 0 and programs <= 2048 runs as a work queue (one workgroup
 * per CU taking the (task, split) units in use, instead of a grid of mostly empty
 * workgroups); the outputs are the same bits. Launches that overlap on one device must not
 * share counters.
 * max_query_len: host upper bound on query tokens per request (0 = unknown). Only
 * min(query_tile, max_query_len) * (hq / H) rows per task are computed, so a decode step
 * (max_query_len 1) does not pay for the query_tile padding; it must not undercount.
 */
int oscar_attention_partials(const void* query, int64_t q_s0, int64_t q_s1, int64_t q_s2,
                             const void* key, int64_t k_s0, int64_t k_s1, int64_t k_s2,
                             const void* value, int64_t v_s0, int64_t v_s1, int64_t v_s2,
                             const void* history, int64_t history_bytes, const void* window,
                             int64_t window_elems, const int32_t* qstarts,
                             const int32_t* seq_lens, const int32_t* block_tables,
                             int64_t table_stride, int64_t table_columns, const int32_t* counts,
                             const int32_t* tasks, const int32_t* task_count, int64_t n,
                             int64_t hq, int64_t programs, int32_t splits, int32_t block_n,
                             int32_t query_tile, int32_t max_query_len, float scale, int32_t raw,
                             int32_t split_tokens, const oscar_layout* layout, float* partials,
                             float* lse, int32_t* queue_counters, void* stream);

/*
 * merge_splits -- replaces kernels.py:506-511 `merge_splits(partials, lse, counts)`.
 * out[t, q, :] = sum_s e^{lse_s - M} P_s / sum_s e^{lse_s - M} (bf16) and
 * logsum[t, q] = M + log(sum) or -inf; rows t >= counts[1] become 0 / -inf.
 */
int oscar_merge_splits(const float* partials, const float* lse, const int32_t* counts, int64_t n,
                       int64_t hq, int32_t splits, int32_t d, void* out, float* logsum,
                       void* stream);

/*
 * merge_paths -- replaces kernels.py:530-541 `merge_paths(history_out, history_lse,
 * raw_partials, raw_lse, counts, output)`.
 * output[t, q*256:(q+1)*256] = (wa*a + wb*b) / (wa + wb), wa = e^{la-M}, wb = e^{lb-M}.
 * history_out: bf16 [n, hq, 256]; raw_partials: fp32 [n, hq, 1, 256]; output: bf16
 * [n, hq*256]. merged_lse (optional, fp32 [n, hq]) = M + log(wa + wb) -- an addition of
 * this library; the reference stores no merged LSE.
 */
int oscar_merge_paths(const void* history_out, const float* history_lse,
                      const float* raw_partials, const float* raw_lse, const int32_t* counts,
                      int64_t n, int64_t hq, int32_t d, void* output, float* merged_lse,
                      void* stream);

/*
 * store_windows -- replaces kernels.py:598-620 `store_windows(key, value, window, meta,
 * layout)`. Writes the current BF16 K/V of each request < counts[0] into its sink
 * slots (position < S) and ring slots (S + position % C, latest writer only) of the
 * owner page (block_tables[req, 0] / (Bp / BK)). Must run after both attention
 * branches of the step. Reference grid: min(n, max_reqs) requests.
 */
int oscar_store_windows(const void* key, int64_t k_s0, int64_t k_s1, int64_t k_s2,
                        const void* value, int64_t v_s0, int64_t v_s1, int64_t v_s2, int64_t n,
                        void* window, int64_t window_elems, const int32_t* qstarts,
                        const int32_t* seq_lens, const int32_t* block_tables,
                        int64_t table_stride, const int32_t* counts, int64_t max_reqs,
                        const oscar_layout* layout, void* stream);

/*
 * unpack -- the dequant half of kernels.py:651-672 `dequant_inverse_rotate(history, slots,
 * rk, rv, layout)` (kernels.py:623-648). key_out/value_out: contiguous bf16 [n, H, 256]
 * with bf16(code * scale + zero); rows with slot < 0 become zeros. n <= 4096.
 */
int oscar_unpack(const void* history, int64_t history_bytes, const int64_t* slots, int64_t n,
                 const oscar_layout* layout, void* key_out, void* value_out, void* stream);

/*
 * pre_attention -- the first of the two fused launches around the history kernel; it has
 * no single counterpart in the reference, it replaces backend.py:171-173 + 195 + 211-222
 * (oscar_ascend/backend.py): `rotate(key, Rk)`, `rotate(value, Rv)`, `store_int2(...)`,
 * `rotate(query, Rk)` and `attention_partials(..., splits=1, raw=True)`.
 * Writes raw_partials fp32 [n, hq, 1, 256] / raw_lse [n, hq, 1] (exactly as
 * oscar_attention_partials with raw != 0 and one split), qrot bf16 [n, hq, 256] (exactly as
 * oscar_rotate of query by Rk) and the INT2 slots of the current tokens (exactly as
 * oscar_store_int2 of the rotated K/V). rk_t / rv_t: R_k^T and R_v^T, contiguous bf16
 * [256][256] (rk_t[c][k] = R_k[k][c]). query/key/value rows must be contiguous and 16-byte
 * aligned (row strides in elements, multiples of 8). qrot == NULL leaves the q rotation out
 * (the caller rotates q itself, e.g. with oscar_rotate on another stream, so that the history
 * launch can start while this one runs: the history branch never reads the slots written
 * here). raw_partials and raw_lse both NULL leaves the BF16 branch out (the caller runs it
 * with oscar_chunk_raw_attention, as for long continuation chunks); one of them NULL is
 * OSCAR_E_NULL.
 */
int oscar_pre_attention(const void* query, int64_t q_s0, int64_t q_s1, const void* key,
                        int64_t k_s0, int64_t k_s1, const void* value, int64_t v_s0, int64_t v_s1,
                        const void* window, int64_t window_elems, const int32_t* qstarts,
                        const int32_t* seq_lens, const int32_t* block_tables,
                        int64_t table_stride, int64_t table_columns, const int32_t* counts,
                        const int32_t* tasks, const int32_t* task_count, int64_t n, int64_t hq,
                        int64_t programs, int32_t block_n, int32_t query_tile,
                        int32_t max_query_len, float scale, const void* rk_t, const void* rv_t,
                        void* history, int64_t history_bytes, const int64_t* slots,
                        const oscar_clip* clip, const oscar_layout* layout, float* raw_partials,
                        float* raw_lse, void* qrot, void* stream);

/*
 * post_attention -- the second fused launch; it replaces backend.py:209-210 + 223-226
 * (oscar_ascend/backend.py): `merge_splits(hp, hl, counts)`, `rotate(hrot, Rv.T)`,
 * `merge_paths(...)` and `store_windows(...)`, in that order of dependence, with the same
 * bits as those entry points. rv: R_v row-major bf16 [256][256]. output: bf16 [n, hq*256];
 * merged_lse (optional): fp32 [n, hq]. The window store runs in workgroups of its own beside
 * the merges; both attention branches read the window in the earlier launches of the step,
 * so this launch must follow the history launch of the same step on the stream.
 */
int oscar_post_attention(const float* history_partials, const float* history_lse,
                         int32_t splits, const float* raw_partials, const float* raw_lse,
                         const int32_t* counts, const void* rv, int64_t n, int64_t hq,
                         void* output, float* merged_lse, const void* key, int64_t k_s0,
                         int64_t k_s1, const void* value, int64_t v_s0, int64_t v_s1,
                         void* window, int64_t window_elems, const int32_t* qstarts,
                         const int32_t* seq_lens, const int32_t* block_tables,
                         int64_t table_stride, int64_t max_reqs, const oscar_layout* layout,
                         void* stream);

/*
 * prefill_attention -- initial prefill (every request's history empty): replaces the
 * reference's fused-infer call (oscar_ascend/backend.py:175-193: causal attention of each
 * request over its own current tokens, output rows past num_actual_tokens zeroed). A flash
 * kernel: 192 (query, head) rows per workgroup share each 32-token K/V block through LDS. Each
 * row has the bits the BF16 branch of oscar_attention_partials (raw, one split) followed by
 * merge_splits + rotate + merge_paths gives a row whose history branch is empty; output: bf16
 * [n, hq*256] (16-byte aligned), merged_lse (optional): fp32 [n, hq]. query: bf16 [n][hq][256],
 * key/value: bf16 [n][kv_heads][256] (row strides in elements, multiples of 8; rows 16-byte
 * aligned). qstarts [max_reqs + 1], seq_lens [max_reqs], counts [2] (live requests, tokens) as
 * for the other entry points; max_query_len: host bound on query tokens per request (0 =
 * unknown: n). Rows of tokens at or past counts[1] are zeroed (LSE -inf). A request whose
 * seq_len differs from its query tokens has history and is not served: its rows are NaN.
 */
int oscar_prefill_attention(const void* query, int64_t q_s0, int64_t q_s1, const void* key,
                            int64_t k_s0, int64_t k_s1, const void* value, int64_t v_s0,
                            int64_t v_s1, const int32_t* qstarts, const int32_t* seq_lens,
                            const int32_t* counts, int64_t n, int64_t hq, int64_t max_reqs,
                            int32_t max_query_len, float scale, const oscar_layout* layout,
                            void* output, float* merged_lse, void* stream);

/*
 * chunk_raw_attention -- the BF16 branch of kernels.py:439-482 (`attention_partials(..., 1,
 * raw=True)`, oscar_ascend/kernels.py: each query row over the sink and recent rows of the
 * request's window page, then its chunk's current tokens causally) as the flash kernel of
 * oscar_prefill_attention, for continuation chunks of many query tokens: the rows of 32
 * consecutive query tokens of a request share each 32-key block through LDS. Writes
 * raw_partials fp32 [n, hq, 1, 256] (16-byte aligned) and raw_lse [n, hq, 1] with the bits of
 * oscar_attention_partials (raw != 0, one split); rows of tokens at or past counts[1] are not
 * written. Arguments as for oscar_pre_attention (window, block table and layout locate each
 * request's window page; max_query_len: host bound on query tokens per request, 0 = n). A
 * request with fewer tokens than query tokens gets NaN rows. A window page that does not lie
 * wholly inside the window buffer contributes no rows (the decode path drops such rows one by
 * one; the two agree whenever the buffer holds whole pages).
 */
int oscar_chunk_raw_attention(const void* query, int64_t q_s0, int64_t q_s1, const void* key,
                              int64_t k_s0, int64_t k_s1, const void* value, int64_t v_s0,
                              int64_t v_s1, const void* window, int64_t window_elems,
                              const int32_t* qstarts, const int32_t* seq_lens,
                              const int32_t* block_tables, int64_t table_stride,
                              int64_t table_columns, const int32_t* counts, int64_t n, int64_t hq,
                              int64_t max_reqs, int32_t max_query_len, float scale,
                              const oscar_layout* layout, float* raw_partials, float* raw_lse,
                              void* stream);

/*
 * history_pre -- the history branch (oscar_attention_partials with raw = 0) and the BF16 branch
 * plus K/V INT2 store of oscar_pre_attention (its q rotation excluded) in ONE launch: the
 * pre-attention work runs as extra workgroups dispatched ahead of the history splits, so it
 * leaves the step's critical path. No reference counterpart as one call: it replaces
 * backend.py:171-173 (rotate K/V, store_int2) and 211-222 (BF16 branch) beside the history
 * attention_partials of backend.py:195-205. query_rot: the rotated query (as for
 * oscar_attention_partials), or NULL: then each history workgroup rotates its task's query rows
 * by R_k itself (the bits of oscar_rotate, so the q rotation of backend.py:195 needs no launch
 * of its own; r_s0..r_s2 are ignored); query/key/value/window/rk_t/rv_t/slots/clip/
 * raw_partials/raw_lse: as for oscar_pre_attention; partials/lse/splits/split_tokens: as for
 * oscar_attention_partials. All outputs have the bits of those two calls. Coverage: query rows
 * per task (min(query_tile, max_query_len) * hq / kv_heads) <= 8, else OSCAR_E_UNSUPPORTED.
 */
int oscar_history_pre(const void* query_rot, int64_t r_s0, int64_t r_s1, int64_t r_s2,
                      const void* query, int64_t q_s0, int64_t q_s1, const void* key,
                      int64_t k_s0, int64_t k_s1, const void* value, int64_t v_s0, int64_t v_s1,
                      void* history, int64_t history_bytes, const void* window,
                      int64_t window_elems, const int32_t* qstarts, const int32_t* seq_lens,
                      const int32_t* block_tables, int64_t table_stride, int64_t table_columns,
                      const int32_t* counts, const int32_t* tasks, const int32_t* task_count,
                      int64_t n, int64_t hq, int64_t programs, int32_t splits, int32_t block_n,
                      int32_t query_tile, int32_t max_query_len, float scale,
                      int32_t split_tokens, const void* rk_t, const void* rv_t,
                      const int64_t* slots, const oscar_clip* clip, const oscar_layout* layout,
                      float* partials, float* lse, float* raw_partials, float* raw_lse,
                      void* stream);

/*
 * history_pre_queue -- oscar_history_pre for 17-32 query rows per task (MTP verification:
 * query_tile x hq / kv_heads rows): the history branch as the work queue of token-bounded
 * (task, split) units (split_tokens != 0; at most 512 task rows, `programs`) with the BF16
 * branch of each (task, kv head) and the K/V store as units of the queue. No reference
 * counterpart as one call: it replaces backend.py:171-173 and 211-222 beside the history
 * attention_partials of backend.py:195-205 for these steps, with the bits of
 * oscar_pre_attention (without its q rotation) and oscar_attention_partials (raw = 0, with the
 * same queue counters). query_rot: the rotated query (required). queue_counters: int32 [2],
 * zero at rest and left zero, as for oscar_attention_partials. Other rows per task, or
 * split_tokens == 0, or more task rows: OSCAR_E_UNSUPPORTED. Calls that overlap on one
 * device must not share the counters.
 */
int oscar_history_pre_queue(const void* query_rot, int64_t r_s0, int64_t r_s1, int64_t r_s2,
                            const void* query, int64_t q_s0, int64_t q_s1, const void* key,
                            int64_t k_s0, int64_t k_s1, const void* value, int64_t v_s0,
                            int64_t v_s1, void* history, int64_t history_bytes,
                            const void* window, int64_t window_elems, const int32_t* qstarts,
                            const int32_t* seq_lens, const int32_t* block_tables,
                            int64_t table_stride, int64_t table_columns, const int32_t* counts,
                            const int32_t* tasks, const int32_t* task_count, int64_t n,
                            int64_t hq, int64_t programs, int32_t splits, int32_t block_n,
                            int32_t query_tile, int32_t max_query_len, float scale,
                            int32_t split_tokens, const void* rk_t, const void* rv_t,
                            const int64_t* slots, const oscar_clip* clip,
                            const oscar_layout* layout, float* partials, float* lse,
                            float* raw_partials, float* raw_lse, int32_t* queue_counters,
                            void* stream);

/*
 * history_pre_q -- oscar_history_pre with the q rotation of backend.py:195 as role workgroups
 * of the same launch (no reference counterpart as one call; it replaces oscar_rotate(query,
 * R_k) followed by oscar_history_pre, with their bits). qrot: bf16 [n, hq, 256] contiguous,
 * receives rotate(query, R_k); the history workgroups read it once the rotation roles are
 * done. qsync: int32 [4], all zero before the first call; each launch leaves it zero (the
 * workgroup that completes the grid resets it). After the launch qsync[2] != 0 means that a
 * history workgroup stopped waiting for the rotation roles (about a millisecond) and its rows
 * are wrong; it never happens when the launch has the device to itself. Calls that overlap on
 * one device with the same qsync race. Other arguments and coverage: as oscar_history_pre.
 */
int oscar_history_pre_q(void* qrot, int32_t* qsync, const void* query, int64_t q_s0,
                        int64_t q_s1, const void* key, int64_t k_s0, int64_t k_s1,
                        const void* value, int64_t v_s0, int64_t v_s1, void* history,
                        int64_t history_bytes, const void* window, int64_t window_elems,
                        const int32_t* qstarts, const int32_t* seq_lens,
                        const int32_t* block_tables, int64_t table_stride, int64_t table_columns,
                        const int32_t* counts, const int32_t* tasks, const int32_t* task_count,
                        int64_t n, int64_t hq, int64_t programs, int32_t splits, int32_t block_n,
                        int32_t query_tile, int32_t max_query_len, float scale,
                        int32_t split_tokens, const void* rk_t, const void* rv_t,
                        const int64_t* slots, const oscar_clip* clip, const oscar_layout* layout,
                        float* partials, float* lse, float* raw_partials, float* raw_lse,
                        void* stream);

/*
 * history_post -- the history branch and post_attention in ONE launch (no reference
 * counterpart: it replaces oscar_attention_partials(raw = 0) followed by
 * oscar_post_attention, with the same output and merged_lse bits). The arguments are those of
 * the two calls (query = the rotated query; partials / lse: fp32 [n, hq, splits, 256] /
 * [n, hq, splits] scratch rows of the launch). The workgroup that completes a (task, kv head)
 * merges that task's rows; counters: int32 [counter_slots >= programs * kv_heads], all zero
 * before the first call, left zero by every call. Calls that overlap on one device must not
 * share counters. Supports query rows per task (min(query_tile, max_query_len) * hq / kv_heads)
 * <= 8 and splits <= 16 (OSCAR_E_UNSUPPORTED otherwise: use the two calls). Split slots a
 * token-bounded request does not use are left unwritten. Must follow oscar_pre_attention of
 * the same step on the stream (it reads raw_partials / raw_lse and stores the windows).
 */
int oscar_history_post(const void* query, int64_t q_s0, int64_t q_s1, int64_t q_s2,
                       const void* history, int64_t history_bytes, const int32_t* qstarts,
                       const int32_t* seq_lens, const int32_t* block_tables,
                       int64_t table_stride, int64_t table_columns, const int32_t* counts,
                       const int32_t* tasks, const int32_t* task_count, int64_t n, int64_t hq,
                       int64_t programs, int32_t splits, int32_t block_n, int32_t query_tile,
                       int32_t max_query_len, float scale, int32_t split_tokens,
                       const oscar_layout* layout, float* partials, float* lse,
                       int32_t* counters, int64_t counter_slots, const float* raw_partials,
                       const float* raw_lse, const void* rv, void* output, float* merged_lse,
                       const void* key, int64_t k_s0, int64_t k_s1, const void* value,
                       int64_t v_s0, int64_t v_s1, void* window, int64_t window_elems,
                       int64_t max_reqs, void* stream);

/*
 * layer_step -- one FULL-attention layer step in ONE launch (no reference counterpart: it
 * replaces the whole sequence of backend.py:171-226 -- rotate K, V and q, store_int2, the
 * history and BF16 attention branches, merge_splits, rotate(hrot, Rv.T), merge_paths and
 * store_windows -- for decode and MTP-verification steps). query/key/value: the step's
 * UNROTATED bf16 rows (row strides in elements, multiples of 8, rows 16-byte aligned);
 * history/window: the K/V stripe views (both written: the INT2 slots of the step's tokens and
 * the windows); rk_t / rv_t: R_k^T and R_v^T, contiguous bf16 [256][256]; rv: R_v row-major.
 * Scratch: partials / lse (fp32 [n, hq, splits, 256] / [n, hq, splits]), raw_partials /
 * raw_lse (fp32 [n, hq, 4, 256] / [n, hq, 4]) and counters (int32 [counter_slots >= programs *
 * kv_heads], zero before the first call, left zero by every call; calls that overlap on one
 * device must not share them). output: bf16 [n, hq * 256]; merged_lse optional fp32 [n, hq].
 * The INT2 bytes and window bytes are those of the single entry points; the output and merged
 * LSE agree with them within rounding (the BF16 branch is merged from up to four splits).
 * Coverage (else OSCAR_E_UNSUPPORTED: use the three fused launches): query rows per task
 * (max_query_len * hq / kv_heads) <= 8, 1 <= max_query_len <= query_tile <= 4 (one task per
 * request), splits <= 16.
 */
int oscar_layer_step(const void* query, int64_t q_s0, int64_t q_s1, const void* key, int64_t k_s0,
                     int64_t k_s1, const void* value, int64_t v_s0, int64_t v_s1, void* history,
                     int64_t history_bytes, void* window, int64_t window_elems,
                     const int32_t* qstarts, const int32_t* seq_lens, const int32_t* block_tables,
                     int64_t table_stride, int64_t table_columns, const int32_t* counts,
                     const int32_t* tasks, const int32_t* task_count, const int64_t* slots,
                     int64_t n, int64_t hq, int64_t programs, int32_t splits, int32_t block_n,
                     int32_t query_tile, int32_t max_query_len, float scale,
                     int32_t split_tokens, const void* rk_t, const void* rv_t, const void* rv,
                     const oscar_clip* clip, const oscar_layout* layout, float* partials,
                     float* lse, float* raw_partials, float* raw_lse, int32_t* counters,
                     int64_t counter_slots, void* output, float* merged_lse, int64_t max_reqs,
                     void* stream);

/*
 * history_post_noalloc -- oscar_history_post without caller scratch: the split partials, their
 * LSEs and the completion counters live in a fixed device array of this library
 * (OSCAR_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends), so the call allocates
 * nothing and needs no workspace argument. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Arguments and results are those of oscar_history_post without
 * partials, lse, counters and counter_slots; the output and merged_lse bits are the same.
 * Limits: oscar_noalloc_scratch_bytes(n, hq, splits) <= OSCAR_NOALLOC_SCRATCH_BYTES and
 * programs * kv_heads <= 16384, else OSCAR_E_SCRATCH (nothing launched). The first call on a
 * device resolves the array's address and clears its counters on `stream`. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (concurrent streams) race.
 */
#define OSCAR_NOALLOC_SCRATCH_BYTES (32ll << 20)

int64_t oscar_noalloc_scratch_bytes(int64_t n, int64_t hq, int32_t splits);

int oscar_history_post_noalloc(const void* query, int64_t q_s0, int64_t q_s1, int64_t q_s2,
                               const void* history, int64_t history_bytes,
                               const int32_t* qstarts, const int32_t* seq_lens,
                               const int32_t* block_tables, int64_t table_stride,
                               int64_t table_columns, const int32_t* counts,
                               const int32_t* tasks, const int32_t* task_count, int64_t n,
                               int64_t hq, int64_t programs, int32_t splits, int32_t block_n,
                               int32_t query_tile, int32_t max_query_len, float scale,
                               int32_t split_tokens, const oscar_layout* layout,
                               const float* raw_partials, const float* raw_lse, const void* rv,
                               void* output, float* merged_lse, const void* key, int64_t k_s0,
                               int64_t k_s1, const void* value, int64_t v_s0, int64_t v_s1,
                               void* window, int64_t window_elems, int64_t max_reqs,
                               void* stream);

/* ---------------------------------------------------------------- calibration (startup) */

/*
 * accumulate_gram -- covariance += sum over rows r = (token, head) of w_r x_r x_r^T
 * (oscar_ascend/calibration_kernels.py:14-70, accumulate_gram). x: [n, heads, dim] bf16
 * (x_fp32 = 0) or fp32 (x_fp32 = 1), element strides s_t, s_h, s_d; weights: fp32 [n * heads]
 * (row index token * heads + head) or NULL for 1; covariance: fp32 [dim, dim] row-major,
 * updated in place. dim a multiple of 32. Deterministic (fixed summation order).
 */
int oscar_accumulate_gram(const void* x, int32_t x_fp32, int64_t n, int64_t heads, int64_t dim,
                          int64_t s_t, int64_t s_h, int64_t s_d, const float* weights,
                          float* covariance, void* stream);

/*
 * sst_weights -- weights[t] = max(k_t^T C_q k_t, 0) for the n key rows of one KV head, and
 * *total_weight += their sum (calibration_kernels.py:73-126, sst_weights). key: bf16 or fp32
 * [n, 1, 256] with element strides s_t (token) and s_d; q_covariance: fp32 [256, 256].
 */
int oscar_sst_weights(const void* key, int32_t key_fp32, int64_t n, int64_t dim, int64_t s_t,
                      int64_t s_d, const float* q_covariance, float* weights,
                      float* total_weight, void* stream);

/*
 * normalize -- out = x / max(denominator, 1e-30) over count fp32 values; the denominator is
 * *denominator when that pointer is non-NULL (a device scalar), else `value`
 * (calibration_kernels.py:129-156, normalize).
 */
int oscar_normalize(const float* x, int64_t count, const float* denominator, float value,
                    float* out, void* stream);

/*
 * calibrated_rotations -- eigen-decomposition of `batch` symmetric fp32 [256, 256] covariances
 * by cyclic round-robin Jacobi sweeps, then R = U H Pbr per matrix
 * (calibration_kernels.py:159-327, calibrated_rotations): eigenvalues fp32 [batch, 256]
 * ascending, rotations fp32 [batch, 256, 256]. Sweeps stop per matrix once the relative
 * off-diagonal residual (max |off-diagonal| / max |diagonal|, checked every second sweep and
 * after the last) is below `tolerance`, or after max_sweeps (<= 64). info: fp32 [batch, 2] =
 * (sweeps run, last residual; +inf for a non-finite matrix) -- the caller reads it back and
 * rejects non-converged results. workspace: >= oscar_calibration_workspace_bytes(batch,
 * max_sweeps) bytes of device memory, 16-byte aligned. Three launches, no host round trip.
 */
int64_t oscar_calibration_workspace_bytes(int32_t batch, int32_t max_sweeps);

int oscar_calibrated_rotations(const float* covariances, int32_t batch, int32_t dim,
                               int32_t max_sweeps, float tolerance, void* workspace,
                               int64_t workspace_bytes, float* rotations, float* eigenvalues,
                               float* info, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OSCAR_HIP_H_ */
