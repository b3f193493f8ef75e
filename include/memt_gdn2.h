/*
 * memt_gdn2.h -- C ABI of the MI355X (gfx950) GDN-2 native-memory hot path.
 *
 * Every entry point takes device pointers, plain sizes and a HIP stream
 * (hipStream_t passed as void*; NULL = the null stream).  None allocates
 * memory, none synchronises the host, and all are reentrant: each call only
 * enqueues kernels on `stream`.  Tensors are token-major and contiguous,
 * exactly as in the reference ([B=1, T, H, D] with the packed token axis
 * first, states [N, H, K, V] fp32).  bf16 is passed as its 16-bit storage.
 *
 * Status: 0 on success, a negative MEMT_GDN2_E* code otherwise
 * (memt_gdn2_strerror names it).  Arguments are validated on the host; a
 * plan (chunk table) is trusted as built by the caller: chunk_len in 1..64,
 * chunk_tok0 + chunk_len within the token axis, offsets non-decreasing.
 */
#ifndef MEMT_GDN2_H
#define MEMT_GDN2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MEMT_GDN2_ABI_VERSION 7

#define MEMT_GDN2_OK 0
#define MEMT_GDN2_EINVAL (-1)       /* null pointer or inconsistent sizes */
#define MEMT_GDN2_EUNSUPPORTED (-2) /* head dim / dtype without a compiled variant */
#define MEMT_GDN2_ELAUNCH (-3)      /* the HIP launch reported an error */
#define MEMT_GDN2_EWORKSPACE (-4)   /* workspace missing or too small */
#define MEMT_GDN2_ESCRATCH (-5)     /* beyond the static scratch of memt_gdn2_chunk_update_noalloc */

/* device scratch of memt_gdn2_chunk_update_noalloc, per GPU (64 MiB) */
#define MEMT_GDN2_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* element types */
#define MEMT_GDN2_F32 0
#define MEMT_GDN2_BF16 1

/* output gate of the readout epilogue */
#define MEMT_GDN2_GATE_SOFTCAP_SILU 0 /* c * tanh(silu(g) / c): MemTRMSNormGated */
#define MEMT_GDN2_GATE_SIGMOID 1      /* sigmoid(g) */

/* memt_gdn2_readout_decode options */
#define MEMT_GDN2_READOUT_L2NORM_Q 1   /* q rows are raw: q_hat = bf16(q / sqrt(sum q^2 + q_eps)) in the kernel */
#define MEMT_GDN2_READOUT_STATE_BF16 2 /* the dot reads bf16(S), as the reference reader does */

/* what the chunked update writes to `o` */
#define MEMT_GDN2_OUT_NONE 0     /* state only */
#define MEMT_GDN2_OUT_SNAPSHOT 1 /* o_t = scale * q_t^T bf16(read_states[seq(t)]) (MemT commit) */
#define MEMT_GDN2_OUT_CAUSAL 2   /* o_t = scale * q_t^T S_t (state after token t) */

/* chunk-plan flag bits */
#define MEMT_GDN2_CHUNK_BLOCK_START 1 /* store a snapshot before this chunk */
#define MEMT_GDN2_CHUNK_COMMIT 2      /* apply this chunk's update */

/*
 * Chunk table: the device-side part of the reference's ChunkPlan
 * (models/qwen/ops/layout.py:18-44).  Chunks are at most 64 tokens and never
 * cross a write event; the decay cumsum restarts at every chunk start.
 */
typedef struct memt_gdn2_plan {
  const int32_t* chunk_tok0;        /* [n_chunk] first token of the chunk on the packed axis */
  const int32_t* chunk_len;         /* [n_chunk] tokens in the chunk, 1..64 */
  const int32_t* seq_chunk_offsets; /* [n_seq + 1] chunk range of each sequence/sample */
  const int32_t* chunk_block_ids;   /* [n_chunk] snapshot (read block) of each chunk, or NULL */
  const int32_t* chunk_flags;       /* [n_chunk] MEMT_GDN2_CHUNK_* bits, or NULL (= commit, no snapshot) */
  int32_t n_chunk;
  int32_t n_seq;
  int32_t n_block; /* rows of `snaps` */
  int32_t reserved;
} memt_gdn2_plan;

/*
 * Host-side chunk plan (no device work, no allocation, no device-to-host copy).
 * Replaces the reference's ChunkPlan builder (models/qwen/ops/layout.py:47-135),
 * which copies its device boundary tensors to the host on every call.
 * Boundaries are host int32 arrays: read [n_read], sample [n_sample] and event
 * [n_event], each non-decreasing from 0 to the same token total.  Every event
 * is cut into chunks of at most wy_tile_tokens (1..64) tokens.
 * memt_gdn2_plan_count writes the chunk count; memt_gdn2_plan_build fills
 * caller-owned host tables of that size: chunk_tok0, chunk_len,
 * chunk_block_ids (the read block of each chunk's first token), chunk_flags
 * (MEMT_GDN2_CHUNK_*), sample_chunk_offsets [n_sample] and, when not NULL,
 * chunk_indices [2 n_chunk] (event, chunk within event), chunk_is_block_start,
 * chunk_commits.  commit_mask [n_event - 1] may be NULL (every event commits).
 */
int memt_gdn2_plan_count(const int32_t* event, int n_event, int wy_tile_tokens, int32_t* n_chunk);
int memt_gdn2_plan_build(const int32_t* read, int n_read, const int32_t* sample, int n_sample,
                         const int32_t* event, int n_event, const uint8_t* commit_mask,
                         int wy_tile_tokens, int32_t n_chunk, int32_t* chunk_tok0,
                         int32_t* chunk_len, int32_t* sample_chunk_offsets,
                         int32_t* chunk_block_ids, int32_t* chunk_flags, int32_t* chunk_indices,
                         int32_t* chunk_is_block_start, int32_t* chunk_commits);

/*
 * Raw projection rows of the memory block (the outputs of its in_proj / f_down
 * GEMMs, read in place): q, k, decay and erase rows hold H*K bf16 channels,
 * v and write rows H*V; each tensor's rows are `*_stride` elements apart
 * (a multiple of 4, at least the row width; pointers 8-byte aligned).
 */
typedef struct memt_gdn2_projections {
  const void* q;
  int64_t q_stride;
  const void* k;
  int64_t k_stride;
  const void* v;
  int64_t v_stride;
  const void* decay; /* f_down(decay latent), pre-softplus */
  int64_t decay_stride;
  const void* erase; /* erase logits */
  int64_t erase_stride;
  const void* write; /* write logits */
  int64_t write_stride;
  const void* decay_bias;      /* [H*K] bf16 */
  const void* decay_scale_log; /* [H] bf16 */
  float eps;                   /* l2norm epsilon (1e-6) */
  int32_t reserved;
} memt_gdn2_projections;

int memt_gdn2_abi_version(void);
const char* memt_gdn2_strerror(int status);

/*
 * Row L2 normalisation y = x / sqrt(sum(x^2) + eps), rstd = 1/sqrt(...).
 * Replaces FLA l2norm_fwd (_vendor/fla/modules/l2norm.py:147-197); dim <= 512.
 * x_dtype/y_dtype: MEMT_GDN2_BF16 or MEMT_GDN2_F32; rstd may be NULL.
 */
int memt_gdn2_l2norm_fwd(const void* x, int x_dtype, void* y, int y_dtype, float* rstd,
                         int64_t rows, int dim, float eps, void* stream);

/*
 * Chunk-local cumulative sum of g [tokens, H, S] over each plan chunk,
 * times `scale` (log2 units when scale = 1/ln 2), fp32 out; `reverse` sums
 * from the chunk end.  Replaces chunk_local_cumsum / chunk_local_cumsum_vector
 * (_vendor/fla/ops/utils/cumsum.py:299-338,444-480) for the [B,T,H,S] layout.
 */
int memt_gdn2_chunk_local_cumsum(const void* g, int g_dtype, float* gk, const memt_gdn2_plan* plan,
                                 int H, int S, float scale, int reverse, void* stream);

/*
 * Bytes of device workspace memt_gdn2_chunk_update (and memt_gdn2_fwd_h, with
 * out_mode NONE) needs for a plan of n_chunk chunks over n_seq sequences.
 * Long sequences get a two-level scan whose group states live here too.
 */
size_t memt_gdn2_chunk_update_workspace_size(int n_chunk, int n_seq, int H, int K, int V, int out_mode);

/*
 * The chunked GDN-2 memory update (stable gated delta rule) end to end:
 * chunk-local decay cumsum, WY/UT transform, inter-chunk fp32 state
 * recurrence and the chosen output.  Replaces token_memory_packed
 * (models/qwen/ops/packed.py:34-81; Flash: models/deepseek/ops/packed.py:70-108)
 * when out_mode = SNAPSHOT, and the FLA chunk GDN-2 forward when CAUSAL.
 *
 *   q, k     [T, H, K] bf16 (q may be NULL when out_mode = NONE)
 *   v        [T, H, V] bf16
 *   g        [T, H, K] fp32 natural-log decay (<= 0)
 *   beta     [T, H, V] write gate, beta_dtype F32 or BF16
 *   b        [T, H, K] bf16 channel erase gate, or NULL for b = 1
 *   h0       [n_seq, H, K, V] fp32 initial states (write_states), or NULL for 0
 *   ht       [n_seq, H, K, V] fp32 final states, or NULL
 *   read_states [n_block, H, K, V] fp32, used by out_mode = SNAPSHOT
 *   snaps    [n_block, H, K, V] fp32 state before each block-start chunk, or NULL
 *   o        [T, H, V] bf16 output (out_mode != NONE)
 * K, V in {64, 128, 256, 512} with K == V; at 512 only MEMT_GDN2_OUT_NONE and
 * MEMT_GDN2_OUT_SNAPSHOT (no causal output).  The workspace must hold
 * memt_gdn2_chunk_update_workspace_size(...) bytes, 256-byte aligned.
 * At K <= 128 the SNAPSHOT read runs inside the state scan when neither ht nor
 * snaps overlaps read_states, and as its own pass ahead of the update otherwise;
 * the output is the same either way, bit for bit.
 */
int memt_gdn2_chunk_update(const void* q, const void* k, const void* v, const float* g,
                           const void* beta, int beta_dtype, const void* b, const float* h0,
                           float* ht, const float* read_states, float* snaps, void* o,
                           const memt_gdn2_plan* plan, int64_t T, int H, int K, int V, float scale,
                           int out_mode, void* workspace, size_t workspace_bytes, void* stream);

/*
 * memt_gdn2_chunk_update without a workspace argument and without allocating:
 * the workspace is the library's own static device scratch of
 * MEMT_GDN2_NOALLOC_SCRATCH_BYTES per GPU (its address is looked up once per
 * device, on the first call with that device current).  It has no counterpart
 * in the reference; it serves callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Returns MEMT_GDN2_ESCRATCH when
 * memt_gdn2_chunk_update_workspace_size(...) exceeds the scratch (about 900
 * 64-token chunk-heads at d = 128 with the causal output).  Every call on one
 * GPU uses the same scratch: calls that overlap on one GPU (concurrent
 * streams) race and must be serialised by the caller.  Arguments and results
 * are those of memt_gdn2_chunk_update.
 */
int memt_gdn2_chunk_update_noalloc(const void* q, const void* k, const void* v, const float* g,
                                   const void* beta, int beta_dtype, const void* b, const float* h0,
                                   float* ht, const float* read_states, float* snaps, void* o,
                                   const memt_gdn2_plan* plan, int64_t T, int H, int K, int V,
                                   float scale, int out_mode, void* stream);

/*
 * memt_gdn2_chunk_update on a pool of state slots, in place: no gather of the
 * states before the call and no scatter of the final states after it.
 * Replaces the executor's torch.cat gather and index_copy_ write-back around
 * the memory block (runtime/executor.py:86-110).
 *   pool     [n_slots, H, K, V] fp32
 *   h0_slot  [n_seq] slot of each sequence's initial state (write_states)
 *   ht_slot  [n_seq] slot that receives each sequence's final state
 *   read_slot [n_block] slot each read block reads (out_mode = SNAPSHOT)
 * A final state may go to the slot its initial state or its read comes from:
 * the read completes before the update starts, and every initial state is
 * read before any final state is written.  Distinct sequences must not share
 * a ht_slot.  Slot indices are trusted (0 <= slot < n_slots).
 */
int memt_gdn2_chunk_update_slots(const void* q, const void* k, const void* v, const float* g,
                                 const void* beta, int beta_dtype, const void* b, float* pool,
                                 int n_slots, const int32_t* read_slot, const int32_t* h0_slot,
                                 const int32_t* ht_slot, void* o, const memt_gdn2_plan* plan, int64_t T,
                                 int H, int K, int V, float scale, int out_mode, void* workspace,
                                 size_t workspace_bytes, void* stream);

/*
 * The commit path of QwenMemoryBlock.packed from its raw projections in one
 * update: the gate and q/k prologue (models/qwen/layer.py:71-97) runs inside
 * the WY kernel (g = -exp(s_h) softplus(decay + bias), beta = bf16(sigmoid(write)),
 * q_hat = l2norm(q), k_til = bf16(sqrt_b * l2norm(k)), unit erase gate), so no
 * prologue tensor goes through HBM.  q_hat [T,H,K] bf16 receives l2norm(q)
 * (required for out_mode SNAPSHOT, which reads it).  States as in
 * memt_gdn2_chunk_update, or, when h0_slot / ht_slot (and read_slot) are not
 * NULL, a pool of n_slots states addressed as in memt_gdn2_chunk_update_slots
 * (h0, ht and read_states then name the same pool).  Also the Flash block's
 * commit (models/deepseek/layer.py:153-183, the same gate and q/k formulas)
 * at K = V = 512, without the causal output.
 */
int memt_gdn2_chunk_update_fused(const memt_gdn2_projections* x, void* q_hat, const float* h0, float* ht,
                                 const float* read_states, int n_slots, const int32_t* read_slot,
                                 const int32_t* h0_slot, const int32_t* ht_slot, void* o,
                                 const memt_gdn2_plan* plan, int64_t T, int H, int K, int V, float scale,
                                 int out_mode, void* workspace, size_t workspace_bytes, void* stream);

/*
 * WY stage only (replaces chunk_gdn2_fwd_intra, _vendor/fla/ops/gdn2/chunk_intra.py:693-787),
 * writing the reference layouts: w, kg [T,H,K] bf16, u [T,H,V] bf16, Akk [T,H,64] bf16
 * (the inverse (I+L)^-1), Aqk [T,H,64] bf16 (scale included; needs q), qg [T,H,K] bf16
 * (q * 2^gk, optional).  gk is the chunk-local cumulative decay in log2 units.
 * Any output pointer may be NULL.  Uses the same workspace as memt_gdn2_chunk_update
 * with out_mode = CAUSAL when q is given, else NONE.
 */
int memt_gdn2_wy_fwd(const void* q, const void* k, const void* v, const float* gk, const void* b,
                     const void* beta, int beta_dtype, const memt_gdn2_plan* plan, int64_t T, int H,
                     int K, int V, float scale, void* w, void* u, void* kg, void* Akk, void* Aqk,
                     void* qg, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Inter-chunk state scan from reference-layout WY tensors (replaces
 * memt_gdn2_fwd_h, models/qwen/ops/_triton/state.py:127-174):
 *   kg, w [T,H,K] bf16, u [T,H,V] bf16, gk [T,H,K] fp32 (log2 cumsum),
 *   h0 [n_seq,H,K,V] or NULL, snaps [n_block,H,K,V] or NULL, ht [n_seq,H,K,V] or NULL.
 * Snapshots are stored before every chunk flagged BLOCK_START; chunks without
 * COMMIT leave the state unchanged.  Uses the chunk_update workspace (out_mode NONE).
 */
int memt_gdn2_fwd_h(const void* kg, const void* w, const void* u, const float* gk,
                    const memt_gdn2_plan* plan, int64_t T, int H, int K, int V, const float* h0,
                    float* snaps, float* ht, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Snapshot reader: o[t] = bf16(scale * q[t]^T bf16(snaps[block(chunk(t))])), fp32
 * accumulation.  Replaces memt_gdn2_read_fwd (models/qwen/ops/read.py:10-39,
 * models/qwen/ops/_triton/read.py:22-71).  q [T,H,K] bf16, snaps [n_block,H,K,V] fp32,
 * o [T,H,V] bf16; plan.chunk_block_ids required.
 */
int memt_gdn2_read_fwd(const void* q, const float* snaps, void* o, const memt_gdn2_plan* plan,
                       int64_t T, int H, int K, int V, float scale, void* stream);

/*
 * memt_gdn2_read_fwd reading block b's state from pool slot read_slot[b]
 * (pool [n_slots, H, K, V] fp32, read_slot [n_block] trusted in range): the
 * query path without the executor's torch.cat gather (runtime/executor.py:86-91).
 */
int memt_gdn2_read_fwd_slots(const void* q, const float* pool, int n_slots, const int32_t* read_slot,
                             void* o, const memt_gdn2_plan* plan, int64_t T, int H, int K, int V,
                             float scale, void* stream);

/*
 * MemTRMSNormGated (models/qwen/layer.py:15-31): for each row of x [rows, dim] bf16,
 * y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w); out = bf16(y * gate_fn(gate)),
 * gate_fn = softcap * tanh(silu(.) / softcap) or sigmoid.  gate [rows, dim] bf16,
 * weight [dim] bf16, dim <= 1024.
 */
int memt_gdn2_rms_norm_gated(const void* x, const void* gate, const void* weight, void* out,
                             int64_t rows, int dim, float eps, float softcap, int gate_kind,
                             void* stream);

/*
 * Fused decode readout: for each sequence b and head h,
 *   r   = bf16(scale * q[b,h]^T S[slot(b),h])       (fp32 state, fp32 accumulation)
 *   out = MemTRMSNormGated(r, gate[b,h]) as above   ([B, H*V] bf16)
 * S [slots, H, K, V] fp32; slot_idx [B] int32 or NULL (slot = b); q [B,H,K] bf16;
 * gate [B,H,V] bf16; weight [V] bf16.  Replaces the query path of
 * QwenMemoryBlock.packed (models/qwen/layer.py:112-131): memt_gdn2_read_fwd + o_norm.
 */
int memt_gdn2_readout_fused(const float* S, const int32_t* slot_idx, const void* q,
                            const void* gate, const void* weight, void* out, int B, int H, int K,
                            int V, float scale, float eps, float softcap, int gate_kind,
                            void* stream);

/*
 * The decode query path of the memory block in one kernel: for each query
 * row b (one token per sample) and head h,
 *   q_hat = l2norm(q[b,h])            (with MEMT_GDN2_READOUT_L2NORM_Q; else q is used as given)
 *   r     = bf16(scale * q_hat^T S)   (S = state[slot(b),h]; bf16(S) with MEMT_GDN2_READOUT_STATE_BF16)
 *   out   = MemTRMSNormGated(r, gate[b,h])   as memt_gdn2_readout_fused
 * q [B, q_stride] bf16 rows holding H*K channels (a view of the fused QKV
 * projection is read in place), gate [B, gate_stride] bf16 rows of H*V
 * channels (strides in elements, at least the row width); S [slots, H, K, V] fp32,
 * slot_idx [B] or NULL (slot = b).  Replaces the query path of
 * QwenMemoryBlock.packed for length-1 samples (models/qwen/layer.py:112-131:
 * l2norm -> memt_gdn2_read_fwd -> o_norm) and of the Flash block
 * (models/deepseek/layer.py:174-183, snapshot_read with
 * bf16_accumulator_output=True -> o_norm).
 */
int memt_gdn2_readout_decode(const float* S, const int32_t* slot_idx, const void* q, int64_t q_stride,
                             const void* gate, int64_t gate_stride, const void* weight, void* out, int B,
                             int H, int K, int V, float scale, float q_eps, float eps, float softcap,
                             int gate_kind, int flags, void* stream);

/*
 * Write gates of the memory block (models/qwen/layer.py:71-88; Flash:
 * models/deepseek/ops/compiled_tensor_ops.py:54-78 after its projections):
 *   g      [T,H,D] fp32 = -exp(decay_scale_log[h]) * softplus(decay + decay_bias)
 *   sqrt_b [T,H,D] bf16 = exp(0.5 * logsigmoid(erase))
 *   beta   [T,H,D] bf16 = sigmoid(write)
 * decay, erase, write: bf16 rows of H*D channels, `*_stride` elements apart
 * (views of the projection outputs; stride >= H*D, a multiple of 8);
 * decay_bias [H*D] bf16, decay_scale_log [H] bf16.  D in {64, 128, 256, 512}.
 * Inputs and outputs 16-byte aligned.
 */
int memt_gdn2_write_gates(const void* decay, int64_t decay_stride, const void* decay_bias,
                          const void* decay_scale_log, const void* erase, int64_t erase_stride,
                          const void* write, int64_t write_stride, float* g, void* sqrt_b, void* beta,
                          int64_t T, int H, int D, void* stream);

/*
 * The whole prologue of QwenMemoryBlock.packed's commit path
 * (models/qwen/layer.py:71-97, _write_gates + _symmetric_inputs) in one pass:
 * g and beta as memt_gdn2_write_gates, and
 *   q_hat [T,H,D] bf16 = q / sqrt(sum q^2 + eps)                    (l2norm_fwd)
 *   k_til [T,H,D] bf16 = bf16(sqrt_b * bf16(k / sqrt(sum k^2 + eps)))
 * q, k: raw bf16 rows with their own strides, as above.  The update then runs
 * with b = 1 (b = NULL in memt_gdn2_chunk_update), as the reference's
 * torch.ones_like(sqrt_b) erase does.
 */
int memt_gdn2_memory_prologue(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                              const void* decay, int64_t decay_stride, const void* decay_bias,
                              const void* decay_scale_log, const void* erase, int64_t erase_stride,
                              const void* write, int64_t write_stride, void* q_hat, void* k_til,
                              float* g, void* beta, int64_t T, int H, int D, float eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MEMT_GDN2_H */
