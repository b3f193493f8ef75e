// extern "C" entry points of libmemt_gdn2.so (declared in include/memt_gdn2.h).
// Host-side argument checks, workspace carving and kernel dispatch.  No entry
// point allocates memory or synchronises the host.
#include <mutex>

#include "gdn2_internal.h"

using namespace memt;

namespace {

bool supported_kv(int K, int V) { return K == V && (K == 64 || K == 128 || K == 256 || K == 512); }
// d = 512 has no causal output (its model reads memory through the snapshot
// read only)
bool wide_ok(int K, bool causal) { return K <= 256 || !causal; }

int status_of(hipError_t e) { return e == hipSuccess ? MEMT_GDN2_OK : MEMT_GDN2_ELAUNCH; }

bool plan_ok(const memt_gdn2_plan* p) {
  return p != nullptr && p->n_chunk >= 0 && p->n_seq >= 0 &&
         (p->n_chunk == 0 || (p->chunk_tok0 != nullptr && p->chunk_len != nullptr));
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// A bf16 row operand of the prologue: H*D channels per token, rows `stride`
// elements apart, 16-byte vector loads.
bool row_operand_ok(const void* p, int64_t stride, int64_t width) {
  return p != nullptr && aligned16(p) && stride >= width && stride % 8 == 0;
}

int prologue_common(PrologueArgs& a, const void* decay, int64_t decay_stride, const void* decay_bias,
                    const void* decay_scale_log, const void* erase, int64_t erase_stride, const void* write,
                    int64_t write_stride, float* g, void* beta, int64_t T, int H, int D) {
  if (T < 0 || H <= 0) return MEMT_GDN2_EINVAL;
  if (D != 64 && D != 128 && D != 256 && D != 512) return MEMT_GDN2_EUNSUPPORTED;
  const int64_t width = (int64_t)H * D;
  if (T > 0) {
    if (!row_operand_ok(decay, decay_stride, width) || !row_operand_ok(erase, erase_stride, width) ||
        !row_operand_ok(write, write_stride, width))
      return MEMT_GDN2_EINVAL;
    if (decay_bias == nullptr || decay_scale_log == nullptr || !aligned16(decay_bias)) return MEMT_GDN2_EINVAL;
    if (g == nullptr || beta == nullptr || !aligned16(g) || !aligned16(beta)) return MEMT_GDN2_EINVAL;
  }
  a = PrologueArgs{};
  a.decay = (const uint16_t*)decay;
  a.decay_bias = (const uint16_t*)decay_bias;
  a.decay_scale_log = (const uint16_t*)decay_scale_log;
  a.erase = (const uint16_t*)erase;
  a.write = (const uint16_t*)write;
  a.decay_stride = decay_stride;
  a.erase_stride = erase_stride;
  a.write_stride = write_stride;
  a.g_out = g;
  a.beta_out = (uint16_t*)beta;
  a.rows = T * H;
  a.H = H;
  return MEMT_GDN2_OK;
}

}  // namespace

extern "C" {

int memt_gdn2_abi_version(void) { return MEMT_GDN2_ABI_VERSION; }

const char* memt_gdn2_strerror(int status) {
  switch (status) {
    case MEMT_GDN2_OK: return "ok";
    case MEMT_GDN2_EINVAL: return "invalid argument (null pointer or inconsistent sizes)";
    case MEMT_GDN2_EUNSUPPORTED: return "unsupported head dimension or dtype";
    case MEMT_GDN2_ELAUNCH: return "kernel launch failed";
    case MEMT_GDN2_EWORKSPACE: return "workspace missing or too small";
    case MEMT_GDN2_ESCRATCH: return "problem needs more than the static scratch of the no-allocation entry point";
    default: return "unknown status";
  }
}

int memt_gdn2_l2norm_fwd(const void* x, int x_dtype, void* y, int y_dtype, float* rstd, int64_t rows, int dim,
                         float eps, void* stream) {
  if (rows < 0 || dim <= 0) return MEMT_GDN2_EINVAL;
  if (rows > 0 && (x == nullptr || y == nullptr)) return MEMT_GDN2_EINVAL;
  if (dim > 512) return MEMT_GDN2_EUNSUPPORTED;
  if ((x_dtype != MEMT_GDN2_BF16 && x_dtype != MEMT_GDN2_F32) ||
      (y_dtype != MEMT_GDN2_BF16 && y_dtype != MEMT_GDN2_F32))
    return MEMT_GDN2_EUNSUPPORTED;
  return status_of(launch_l2norm(x, x_dtype == MEMT_GDN2_BF16, y, y_dtype == MEMT_GDN2_BF16, rstd, rows, dim, eps,
                                 (hipStream_t)stream));
}

int memt_gdn2_chunk_local_cumsum(const void* g, int g_dtype, float* gk, const memt_gdn2_plan* plan, int H, int S,
                                 float scale, int reverse, void* stream) {
  if (!plan_ok(plan) || H <= 0 || S <= 0) return MEMT_GDN2_EINVAL;
  if (plan->n_chunk > 0 && (g == nullptr || gk == nullptr)) return MEMT_GDN2_EINVAL;
  if (g_dtype != MEMT_GDN2_BF16 && g_dtype != MEMT_GDN2_F32) return MEMT_GDN2_EUNSUPPORTED;
  return status_of(launch_cumsum(g, g_dtype == MEMT_GDN2_BF16, gk, plan->chunk_tok0, plan->chunk_len, plan->n_chunk,
                                 H, S, scale, reverse != 0, (hipStream_t)stream));
}

size_t memt_gdn2_chunk_update_workspace_size(int n_chunk, int n_seq, int H, int K, int V, int out_mode) {
  if (n_chunk < 0 || n_seq < 0 || H <= 0 || K <= 0 || V <= 0) return 0;
  const size_t wy = wy_layout(n_chunk, H, K, V, out_mode == MEMT_GDN2_OUT_CAUSAL).total;
  return group_layout(wy, n_chunk, n_seq, H, K, V, nullptr, nullptr);
}

}  // extern "C"

namespace {

bool raw_row_ok(const void* p, int64_t stride, int64_t width) {
  return p != nullptr && ((uintptr_t)p & 7u) == 0 && stride >= width && stride % 4 == 0;
}

int chunk_update(const void* q, const void* k, const void* v, const float* g, const void* beta, int beta_dtype,
                 const void* b, const float* h0, float* ht, const float* read_states, float* snaps, void* o,
                 const memt_gdn2_plan* plan, int64_t T, int H, int K, int V, float scale, int out_mode,
                 void* workspace, size_t workspace_bytes, void* stream, const int32_t* read_slot,
                 const int32_t* h0_slot, const int32_t* ht_slot, const memt_gdn2_projections* x = nullptr,
                 void* q_hat = nullptr) {
  if (!plan_ok(plan) || T < 0 || H <= 0) return MEMT_GDN2_EINVAL;
  if (x != nullptr) {
    // raw projections: the prologue runs inside the WY kernel
    if (!supported_kv(K, V)) return MEMT_GDN2_EUNSUPPORTED;
    const int64_t wk = (int64_t)H * K, wv = (int64_t)H * V;
    if (plan->n_chunk > 0) {
      if (!raw_row_ok(x->q, x->q_stride, wk) || !raw_row_ok(x->k, x->k_stride, wk) ||
          !raw_row_ok(x->v, x->v_stride, wv) || !raw_row_ok(x->decay, x->decay_stride, wk) ||
          !raw_row_ok(x->erase, x->erase_stride, wk) || !raw_row_ok(x->write, x->write_stride, wv) ||
          x->decay_bias == nullptr || ((uintptr_t)x->decay_bias & 7u) || x->decay_scale_log == nullptr)
        return MEMT_GDN2_EINVAL;
      if (out_mode == MEMT_GDN2_OUT_SNAPSHOT && q_hat == nullptr) return MEMT_GDN2_EINVAL;
    }
    q = x->q;
    k = x->k;
    v = x->v;
    g = (const float*)x->decay;  // placeholders for the checks below; the kernel reads the raw rows
    beta = x->write;
    beta_dtype = MEMT_GDN2_BF16;
    b = nullptr;
  }
  if (!supported_kv(K, V)) return MEMT_GDN2_EUNSUPPORTED;
  if (beta_dtype != MEMT_GDN2_F32 && beta_dtype != MEMT_GDN2_BF16) return MEMT_GDN2_EUNSUPPORTED;
  if (out_mode != MEMT_GDN2_OUT_NONE && out_mode != MEMT_GDN2_OUT_SNAPSHOT && out_mode != MEMT_GDN2_OUT_CAUSAL)
    return MEMT_GDN2_EINVAL;
  if (!wide_ok(K, out_mode == MEMT_GDN2_OUT_CAUSAL)) return MEMT_GDN2_EUNSUPPORTED;
  if (plan->n_chunk > 0) {
    if (k == nullptr || v == nullptr || g == nullptr || beta == nullptr || plan->seq_chunk_offsets == nullptr)
      return MEMT_GDN2_EINVAL;
    if (x == nullptr && (!aligned16(k) || !aligned16(v) || (b && !aligned16(b)) || (q && !aligned16(q))))
      return MEMT_GDN2_EINVAL;
    if (out_mode != MEMT_GDN2_OUT_NONE && (q == nullptr || o == nullptr)) return MEMT_GDN2_EINVAL;
    if (out_mode == MEMT_GDN2_OUT_SNAPSHOT && (read_states == nullptr || plan->chunk_block_ids == nullptr))
      return MEMT_GDN2_EINVAL;
    if (snaps != nullptr && (plan->chunk_flags == nullptr || plan->chunk_block_ids == nullptr))
      return MEMT_GDN2_EINVAL;
  }
  const bool causal = out_mode == MEMT_GDN2_OUT_CAUSAL;
  const WyLayout lay = wy_layout(plan->n_chunk, H, K, V, causal);
  const size_t need = group_layout(lay.total, plan->n_chunk, plan->n_seq, H, K, V, nullptr, nullptr);
  if (plan->n_chunk > 0 && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255u)))
    return MEMT_GDN2_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  const WyBuffers buf = wy_buffers(workspace, lay, causal);

  // d <= 128, snapshot mode: the column-split scan runs the read itself (it reads
  // q_hat with its records and the read state once per workgroup), unless a
  // workgroup of that launch may write the read states: pool slots (whose
  // values the host does not see), snapshots, or final states that overlap them.
  const size_t state_bytes = (size_t)H * K * V * sizeof(float);
  auto overlaps = [](const void* p, size_t np, const void* r, size_t nr) {
    return p != nullptr && r != nullptr && (const char*)p < (const char*)r + nr && (const char*)r < (const char*)p + np;
  };
  const bool fuse_read = out_mode == MEMT_GDN2_OUT_SNAPSHOT && K == V && K <= 128 && plan->n_chunk > 0 &&
                         read_slot == nullptr && ht_slot == nullptr && snaps == nullptr &&
                         !overlaps(read_states, (size_t)plan->n_block * state_bytes, ht,
                                   (size_t)plan->n_seq * state_bytes);

  if (out_mode == MEMT_GDN2_OUT_SNAPSHOT && x == nullptr && !fuse_read) {
    // before the scan: with slots, the read may name the slot the update overwrites
    hipError_t e = launch_read_fwd((const __bf16*)q, read_states, (__bf16*)o, plan->chunk_tok0, plan->chunk_len,
                                   plan->chunk_block_ids, plan->n_chunk, H, K, V, scale, st, read_slot);
    if (e != hipSuccess) return MEMT_GDN2_ELAUNCH;
  }
  WyArgs wa{};
  wa.q = causal ? (const __bf16*)q : nullptr;
  wa.k = (const __bf16*)k;
  wa.v = (const __bf16*)v;
  wa.g = g;
  wa.beta = beta;
  wa.b = (const __bf16*)b;
  wa.chunk_tok0 = plan->chunk_tok0;
  wa.chunk_len = plan->chunk_len;
  wa.H = H;
  wa.scale = scale;
  wa.out = buf;
  wa.A_ref = nullptr;
  if (x != nullptr) {
    wa.q = (const __bf16*)x->q;
    wa.f_raw = (const __bf16*)x->decay;
    wa.e_raw = (const __bf16*)x->erase;
    wa.w_raw = (const __bf16*)x->write;
    wa.decay_bias = (const __bf16*)x->decay_bias;
    wa.decay_scale_log = (const __bf16*)x->decay_scale_log;
    wa.q_hat = (__bf16*)q_hat;
    wa.q_stride = x->q_stride;
    wa.k_stride = x->k_stride;
    wa.v_stride = x->v_stride;
    wa.f_stride = x->decay_stride;
    wa.e_stride = x->erase_stride;
    wa.w_stride = x->write_stride;
    wa.eps = x->eps;
  }
  hipError_t e = launch_wy(wa, plan->n_chunk, K, V, causal, false, beta_dtype == MEMT_GDN2_BF16, st);
  if (e != hipSuccess) return MEMT_GDN2_ELAUNCH;
  if (out_mode == MEMT_GDN2_OUT_SNAPSHOT && x != nullptr && !fuse_read) {
    // q_hat comes from the WY kernel; the read still precedes the scan
    e = launch_read_fwd((const __bf16*)q_hat, read_states, (__bf16*)o, plan->chunk_tok0, plan->chunk_len,
                        plan->chunk_block_ids, plan->n_chunk, H, K, V, scale, st, read_slot);
    if (e != hipSuccess) return MEMT_GDN2_ELAUNCH;
  }

  StateArgs sa{};
  sa.in = buf;
  sa.chunk_tok0 = plan->chunk_tok0;
  sa.chunk_len = plan->chunk_len;
  sa.seq_chunk_offsets = plan->seq_chunk_offsets;
  sa.chunk_block_ids = plan->chunk_block_ids;
  sa.chunk_flags = plan->chunk_flags;
  sa.h0 = h0;
  sa.ht = ht;
  sa.h0_slot = h0 ? h0_slot : nullptr;
  sa.ht_slot = ht ? ht_slot : nullptr;
  sa.snaps = snaps;
  sa.o = (causal || fuse_read) ? (__bf16*)o : nullptr;
  if (fuse_read) {
    sa.rd_states = read_states;
    sa.rd_q = (const __bf16*)(x != nullptr ? q_hat : q);
  }
  sa.H = H;
  sa.n_seq = plan->n_seq;
  sa.n_chunk = plan->n_chunk;
  sa.scale = scale;
  sa.group_L = scan_group_chunks(plan->n_chunk, plan->n_seq, H, V);
  group_layout(lay.total, plan->n_chunk, plan->n_seq, H, K, V, &sa.grp, workspace);
  return status_of(launch_state(sa, K, V, causal, st));
}

// Static scratch of memt_gdn2_chunk_update_noalloc: the chunked update's
// workspace for callers that cannot allocate.  One copy per GPU, held from the
// module's load until the process ends; every call on a GPU reuses it (calls
// that overlap on one GPU race on it).  Its contents need no clearing between
// calls: every workspace byte a call reads was written earlier in that call.
__device__ __align__(256) unsigned char scratch[MEMT_GDN2_NOALLOC_SCRATCH_BYTES];

// Device address of `scratch` on each GPU (the host-side symbol is only a
// stand-in), looked up once per device with that device current.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MEMT_GDN2_ELAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return MEMT_GDN2_ELAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MEMT_GDN2_OK;
}

}  // namespace

extern "C" {

int memt_gdn2_chunk_update(const void* q, const void* k, const void* v, const float* g, const void* beta,
                           int beta_dtype, const void* b, const float* h0, float* ht, const float* read_states,
                           float* snaps, void* o, const memt_gdn2_plan* plan, int64_t T, int H, int K, int V,
                           float scale, int out_mode, void* workspace, size_t workspace_bytes, void* stream) {
  return chunk_update(q, k, v, g, beta, beta_dtype, b, h0, ht, read_states, snaps, o, plan, T, H, K, V, scale,
                      out_mode, workspace, workspace_bytes, stream, nullptr, nullptr, nullptr);
}

int memt_gdn2_chunk_update_noalloc(const void* q, const void* k, const void* v, const float* g, const void* beta,
                                   int beta_dtype, const void* b, const float* h0, float* ht,
                                   const float* read_states, float* snaps, void* o, const memt_gdn2_plan* plan,
                                   int64_t T, int H, int K, int V, float scale, int out_mode, void* stream) {
  if (!plan_ok(plan) || H <= 0 || K <= 0 || V <= 0) return MEMT_GDN2_EINVAL;
  const size_t need = memt_gdn2_chunk_update_workspace_size(plan->n_chunk, plan->n_seq, H, K, V, out_mode);
  if (need > MEMT_GDN2_NOALLOC_SCRATCH_BYTES) return MEMT_GDN2_ESCRATCH;
  void* ws = nullptr;
  const int st = scratch_of_current_device(&ws);
  if (st != MEMT_GDN2_OK) return st;
  return chunk_update(q, k, v, g, beta, beta_dtype, b, h0, ht, read_states, snaps, o, plan, T, H, K, V, scale,
                      out_mode, ws, MEMT_GDN2_NOALLOC_SCRATCH_BYTES, stream, nullptr, nullptr, nullptr);
}

int memt_gdn2_chunk_update_fused(const memt_gdn2_projections* x, void* q_hat, const float* h0, float* ht,
                                 const float* read_states, int n_slots, const int32_t* read_slot,
                                 const int32_t* h0_slot, const int32_t* ht_slot, void* o,
                                 const memt_gdn2_plan* plan, int64_t T, int H, int K, int V, float scale,
                                 int out_mode, void* workspace, size_t workspace_bytes, void* stream) {
  if (x == nullptr) return MEMT_GDN2_EINVAL;
  const bool slots = h0_slot != nullptr || ht_slot != nullptr || read_slot != nullptr;
  if (slots) {
    if (n_slots <= 0 || h0_slot == nullptr || ht_slot == nullptr || h0 == nullptr || h0 != ht) return MEMT_GDN2_EINVAL;
    if (out_mode == MEMT_GDN2_OUT_SNAPSHOT && (read_slot == nullptr || read_states != h0)) return MEMT_GDN2_EINVAL;
  }
  return chunk_update(nullptr, nullptr, nullptr, nullptr, nullptr, MEMT_GDN2_BF16, nullptr, h0, ht, read_states,
                      nullptr, o, plan, T, H, K, V, scale, out_mode, workspace, workspace_bytes, stream,
                      slots && out_mode == MEMT_GDN2_OUT_SNAPSHOT ? read_slot : nullptr, slots ? h0_slot : nullptr,
                      slots ? ht_slot : nullptr, x, q_hat);
}

int memt_gdn2_chunk_update_slots(const void* q, const void* k, const void* v, const float* g, const void* beta,
                                 int beta_dtype, const void* b, float* pool, int n_slots, const int32_t* read_slot,
                                 const int32_t* h0_slot, const int32_t* ht_slot, void* o,
                                 const memt_gdn2_plan* plan, int64_t T, int H, int K, int V, float scale,
                                 int out_mode, void* workspace, size_t workspace_bytes, void* stream) {
  if (pool == nullptr || n_slots <= 0 || h0_slot == nullptr || ht_slot == nullptr) return MEMT_GDN2_EINVAL;
  if (out_mode == MEMT_GDN2_OUT_SNAPSHOT && read_slot == nullptr) return MEMT_GDN2_EINVAL;
  if (!aligned16(pool)) return MEMT_GDN2_EINVAL;
  return chunk_update(q, k, v, g, beta, beta_dtype, b, pool, pool, pool, nullptr, o, plan, T, H, K, V, scale,
                      out_mode, workspace, workspace_bytes, stream,
                      out_mode == MEMT_GDN2_OUT_SNAPSHOT ? read_slot : nullptr, h0_slot, ht_slot);
}

int memt_gdn2_wy_fwd(const void* q, const void* k, const void* v, const float* gk, const void* b, const void* beta,
                     int beta_dtype, const memt_gdn2_plan* plan, int64_t T, int H, int K, int V, float scale, void* w,
                     void* u, void* kg, void* Akk, void* Aqk, void* qg, void* workspace, size_t workspace_bytes,
                     void* stream) {
  if (!plan_ok(plan) || T < 0 || H <= 0) return MEMT_GDN2_EINVAL;
  if (!supported_kv(K, V)) return MEMT_GDN2_EUNSUPPORTED;
  if (beta_dtype != MEMT_GDN2_F32 && beta_dtype != MEMT_GDN2_BF16) return MEMT_GDN2_EUNSUPPORTED;
  if (plan->n_chunk > 0 && (k == nullptr || v == nullptr || gk == nullptr || beta == nullptr)) return MEMT_GDN2_EINVAL;
  if ((Aqk != nullptr || qg != nullptr) && q == nullptr) return MEMT_GDN2_EINVAL;
  const bool causal = q != nullptr;
  if (!wide_ok(K, causal)) return MEMT_GDN2_EUNSUPPORTED;
  const WyLayout lay = wy_layout(plan->n_chunk, H, K, V, causal);
  if (plan->n_chunk > 0 && (workspace == nullptr || workspace_bytes < lay.total || ((uintptr_t)workspace & 255u)))
    return MEMT_GDN2_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  const WyBuffers buf = wy_buffers(workspace, lay, causal);
  WyArgs wa{};
  wa.q = (const __bf16*)q;
  wa.k = (const __bf16*)k;
  wa.v = (const __bf16*)v;
  wa.g = gk;
  wa.beta = beta;
  wa.b = (const __bf16*)b;
  wa.chunk_tok0 = plan->chunk_tok0;
  wa.chunk_len = plan->chunk_len;
  wa.H = H;
  wa.scale = scale;
  wa.out = buf;
  wa.A_ref = (__bf16*)Akk;
  hipError_t e = launch_wy(wa, plan->n_chunk, K, V, causal, true, beta_dtype == MEMT_GDN2_BF16, st);
  if (e != hipSuccess) return MEMT_GDN2_ELAUNCH;
  return status_of(launch_wy_export(buf, plan->chunk_tok0, plan->chunk_len, plan->n_chunk, H, K, V, (__bf16*)w,
                                    (__bf16*)u, (__bf16*)kg, (__bf16*)Aqk, (__bf16*)qg, st));
}

int memt_gdn2_fwd_h(const void* kg, const void* w, const void* u, const float* gk, const memt_gdn2_plan* plan,
                    int64_t T, int H, int K, int V, const float* h0, float* snaps, float* ht, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (!plan_ok(plan) || T < 0 || H <= 0) return MEMT_GDN2_EINVAL;
  if (!supported_kv(K, V)) return MEMT_GDN2_EUNSUPPORTED;
  if (plan->n_chunk > 0 && (kg == nullptr || w == nullptr || u == nullptr || gk == nullptr ||
                            plan->seq_chunk_offsets == nullptr))
    return MEMT_GDN2_EINVAL;
  if (snaps != nullptr && (plan->chunk_flags == nullptr || plan->chunk_block_ids == nullptr)) return MEMT_GDN2_EINVAL;
  const WyLayout lay = wy_layout(plan->n_chunk, H, K, V, false);
  const size_t need = group_layout(lay.total, plan->n_chunk, plan->n_seq, H, K, V, nullptr, nullptr);
  if (plan->n_chunk > 0 && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255u)))
    return MEMT_GDN2_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  const WyBuffers buf = wy_buffers(workspace, lay, false);
  hipError_t e = launch_wy_import((const __bf16*)w, (const __bf16*)u, (const __bf16*)kg, gk, plan->chunk_tok0,
                                  plan->chunk_len, plan->n_chunk, H, K, V, buf, st);
  if (e != hipSuccess) return MEMT_GDN2_ELAUNCH;
  StateArgs sa{};
  sa.in = buf;
  sa.chunk_tok0 = plan->chunk_tok0;
  sa.chunk_len = plan->chunk_len;
  sa.seq_chunk_offsets = plan->seq_chunk_offsets;
  sa.chunk_block_ids = plan->chunk_block_ids;
  sa.chunk_flags = plan->chunk_flags;
  sa.h0 = h0;
  sa.ht = ht;
  sa.snaps = snaps;
  sa.o = nullptr;
  sa.H = H;
  sa.n_seq = plan->n_seq;
  sa.n_chunk = plan->n_chunk;
  sa.scale = 1.f;
  sa.group_L = scan_group_chunks(plan->n_chunk, plan->n_seq, H, V);
  group_layout(lay.total, plan->n_chunk, plan->n_seq, H, K, V, &sa.grp, workspace);
  return status_of(launch_state(sa, K, V, false, st));
}

int memt_gdn2_read_fwd(const void* q, const float* snaps, void* o, const memt_gdn2_plan* plan, int64_t T, int H,
                       int K, int V, float scale, void* stream) {
  if (!plan_ok(plan) || T < 0 || H <= 0) return MEMT_GDN2_EINVAL;
  if (!supported_kv(K, V)) return MEMT_GDN2_EUNSUPPORTED;
  if (plan->n_chunk > 0 && (q == nullptr || snaps == nullptr || o == nullptr || plan->chunk_block_ids == nullptr))
    return MEMT_GDN2_EINVAL;
  if (!aligned16(q) || !aligned16(snaps)) return MEMT_GDN2_EINVAL;
  return status_of(launch_read_fwd((const __bf16*)q, snaps, (__bf16*)o, plan->chunk_tok0, plan->chunk_len,
                                   plan->chunk_block_ids, plan->n_chunk, H, K, V, scale, (hipStream_t)stream));
}

int memt_gdn2_read_fwd_slots(const void* q, const float* pool, int n_slots, const int32_t* read_slot, void* o,
                             const memt_gdn2_plan* plan, int64_t T, int H, int K, int V, float scale, void* stream) {
  if (pool == nullptr || n_slots <= 0 || read_slot == nullptr) return MEMT_GDN2_EINVAL;
  if (!plan_ok(plan) || T < 0 || H <= 0) return MEMT_GDN2_EINVAL;
  if (!supported_kv(K, V)) return MEMT_GDN2_EUNSUPPORTED;
  if (plan->n_chunk > 0 && (q == nullptr || o == nullptr || plan->chunk_block_ids == nullptr)) return MEMT_GDN2_EINVAL;
  if (!aligned16(q) || !aligned16(pool)) return MEMT_GDN2_EINVAL;
  return status_of(launch_read_fwd((const __bf16*)q, pool, (__bf16*)o, plan->chunk_tok0, plan->chunk_len,
                                   plan->chunk_block_ids, plan->n_chunk, H, K, V, scale, (hipStream_t)stream,
                                   read_slot));
}

int memt_gdn2_rms_norm_gated(const void* x, const void* gate, const void* weight, void* out, int64_t rows, int dim,
                             float eps, float softcap, int gate_kind, void* stream) {
  if (rows < 0 || dim <= 0) return MEMT_GDN2_EINVAL;
  if (rows > 0 && (x == nullptr || gate == nullptr || weight == nullptr || out == nullptr)) return MEMT_GDN2_EINVAL;
  if (dim > 1024) return MEMT_GDN2_EUNSUPPORTED;
  if (gate_kind != MEMT_GDN2_GATE_SOFTCAP_SILU && gate_kind != MEMT_GDN2_GATE_SIGMOID) return MEMT_GDN2_EINVAL;
  if (gate_kind == MEMT_GDN2_GATE_SOFTCAP_SILU && !(softcap > 0.f)) return MEMT_GDN2_EINVAL;
  return status_of(launch_rms_norm_gated((const __bf16*)x, (const __bf16*)gate, (const __bf16*)weight, (__bf16*)out,
                                         rows, dim, eps, softcap, gate_kind, (hipStream_t)stream));
}

int memt_gdn2_readout_fused(const float* S, const int32_t* slot_idx, const void* q, const void* gate,
                            const void* weight, void* out, int B, int H, int K, int V, float scale, float eps,
                            float softcap, int gate_kind, void* stream) {
  return memt_gdn2_readout_decode(S, slot_idx, q, (int64_t)H * K, gate, (int64_t)H * V, weight, out, B, H, K, V,
                                  scale, 0.f, eps, softcap, gate_kind, 0, stream);
}

int memt_gdn2_readout_decode(const float* S, const int32_t* slot_idx, const void* q, int64_t q_stride,
                             const void* gate, int64_t gate_stride, const void* weight, void* out, int B, int H,
                             int K, int V, float scale, float q_eps, float eps, float softcap, int gate_kind,
                             int flags, void* stream) {
  if (B < 0 || H <= 0) return MEMT_GDN2_EINVAL;
  if (!supported_kv(K, V)) return MEMT_GDN2_EUNSUPPORTED;
  if (flags & ~(MEMT_GDN2_READOUT_L2NORM_Q | MEMT_GDN2_READOUT_STATE_BF16)) return MEMT_GDN2_EINVAL;
  if (B > 0) {
    if (S == nullptr || q == nullptr || gate == nullptr || weight == nullptr || out == nullptr) return MEMT_GDN2_EINVAL;
    if (q_stride < (int64_t)H * K || gate_stride < (int64_t)H * V) return MEMT_GDN2_EINVAL;
  }
  if (!aligned16(S)) return MEMT_GDN2_EINVAL;
  if (gate_kind != MEMT_GDN2_GATE_SOFTCAP_SILU && gate_kind != MEMT_GDN2_GATE_SIGMOID) return MEMT_GDN2_EINVAL;
  if (gate_kind == MEMT_GDN2_GATE_SOFTCAP_SILU && !(softcap > 0.f)) return MEMT_GDN2_EINVAL;
  ReadoutArgs a{};
  a.S = S;
  a.slot_idx = slot_idx;
  a.q = (const __bf16*)q;
  a.gate = (const __bf16*)gate;
  a.weight = (const __bf16*)weight;
  a.out = (__bf16*)out;
  a.q_stride = q_stride;
  a.gate_stride = gate_stride;
  a.H = H;
  a.flags = flags;
  a.scale = scale;
  a.q_eps = q_eps;
  a.eps = eps;
  a.softcap = softcap;
  a.gate_kind = gate_kind;
  return status_of(launch_readout(a, B, K, V, (flags & MEMT_GDN2_READOUT_STATE_BF16) != 0, (hipStream_t)stream));
}

int memt_gdn2_write_gates(const void* decay, int64_t decay_stride, const void* decay_bias,
                          const void* decay_scale_log, const void* erase, int64_t erase_stride, const void* write,
                          int64_t write_stride, float* g, void* sqrt_b, void* beta, int64_t T, int H, int D,
                          void* stream) {
  PrologueArgs a;
  const int st = prologue_common(a, decay, decay_stride, decay_bias, decay_scale_log, erase, erase_stride, write,
                                 write_stride, g, beta, T, H, D);
  if (st != MEMT_GDN2_OK) return st;
  if (T > 0 && (sqrt_b == nullptr || !aligned16(sqrt_b))) return MEMT_GDN2_EINVAL;
  a.erase_out = (uint16_t*)sqrt_b;
  return status_of(launch_prologue(a, D, false, (hipStream_t)stream));
}

int memt_gdn2_memory_prologue(const void* q, int64_t q_stride, const void* k, int64_t k_stride, const void* decay,
                              int64_t decay_stride, const void* decay_bias, const void* decay_scale_log,
                              const void* erase, int64_t erase_stride, const void* write, int64_t write_stride,
                              void* q_hat, void* k_til, float* g, void* beta, int64_t T, int H, int D, float eps,
                              void* stream) {
  PrologueArgs a;
  const int st = prologue_common(a, decay, decay_stride, decay_bias, decay_scale_log, erase, erase_stride, write,
                                 write_stride, g, beta, T, H, D);
  if (st != MEMT_GDN2_OK) return st;
  if (T > 0) {
    const int64_t width = (int64_t)H * D;
    if (!row_operand_ok(q, q_stride, width) || !row_operand_ok(k, k_stride, width)) return MEMT_GDN2_EINVAL;
    if (q_hat == nullptr || k_til == nullptr || !aligned16(q_hat) || !aligned16(k_til)) return MEMT_GDN2_EINVAL;
  }
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.q_stride = q_stride;
  a.k_stride = k_stride;
  a.q_out = (uint16_t*)q_hat;
  a.k_out = (uint16_t*)k_til;
  a.eps = eps;
  return status_of(launch_prologue(a, D, true, (hipStream_t)stream));
}

}  // extern "C"
