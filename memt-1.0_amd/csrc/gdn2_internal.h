// Internal declarations of the GDN-2 kernels: workspace layout, fragment
// orders and per-kernel argument blocks.  Not part of the C ABI.
#pragma once

#include "common.h"
#include "../../include/memt_gdn2.h"

namespace memt {

constexpr int kChunk = 64;  // WY tile tokens (models/common/constants.py:3)

// ---------------------------------------------------------------------------
// Fragment orders.  The WY stage writes its outputs already arranged as the
// MFMA operands the state scan loads, so every lane of the scan issues one
// 16-byte (A operand) or 8-byte (C fragment) load and a wave reads a
// contiguous 1 KiB / 512 B span.
//
//  A-frag of X[rows][red] (red % 32 == 0), 8 elements per lane:
//     index = ((rt * red/32 + s) * 64 + lane) * 8 + e
//     <-> X[16*rt + lane%16][32*s + 8*(lane/16) + e]
//  C-frag of X[rows][n] (n % 16 == 0), 4 elements per lane:
//     index = ((rt * n/16 + ct) * 64 + lane) * 4 + e
//     <-> X[16*rt + 4*(lane/16) + e][16*ct + lane%16]
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ int afrag_index(int row, int col, int red) {
  const int rt = row >> 4, s = col >> 5;
  const int lane = (row & 15) + ((col >> 3) & 3) * 16;
  return ((rt * (red >> 5) + s) * 64 + lane) * 8 + (col & 7);
}
// P-frag: an A-frag whose reduction index is permuted so that it pairs with a
// B operand assembled from two C fragments (rows 4*(lane/16)+0..3 of 16-row
// tiles 2s and 2s+1).  Lane l's 8 elements at step s are
//   X[16*rt + l%16][32*s + 4*(l/16) + e]        e = 0..3
//   X[16*rt + l%16][32*s + 16 + 4*(l/16) + e]   e = 0..3
// so accumulators of one product feed the next without an LDS round trip.
__host__ __device__ __forceinline__ int pfrag_index(int row, int col, int red) {
  const int rt = row >> 4, s = col >> 5, within = col & 31;
  const int half = within >> 4, lg = (within & 15) >> 2, e = within & 3;
  const int lane = (row & 15) + lg * 16;
  return ((rt * (red >> 5) + s) * 64 + lane) * 8 + half * 4 + e;
}
__host__ __device__ __forceinline__ int cfrag_index(int row, int col, int n) {
  const int rt = row >> 4, ct = col >> 4;
  const int lane = (col & 15) + ((row >> 2) & 3) * 16;
  return ((rt * (n >> 4) + ct) * 64 + lane) * 4 + (row & 3);
}

__host__ __device__ __forceinline__ size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Per-(chunk, head) records of the WY stage, unit u = chunk * H + head.
//   W     f16  [64 x K]  P-frag (rows = tokens, red = K)       erase path
//   kgT   f16  [K x 64]  P-frag of kg^T (rows = K, red = tokens) value path
//   U     f16  [64 x V]  C-frag                                 value path
//   decay f32  [K]       2^{gk_last}
//   qg    f16  [64 x K]  P-frag, q * 2^{gk}                     (causal output)
//   Aqk   f16  [64 x 64] P-frag, scale * causal scores          (causal output)
//   uexp  i32  [NP]      U is stored as U * 2^-uexp per channel pass (see below)
//
// Value range.  W, kg, qg and Aqk are bounded by |q|, |k| <= 1 (l2-normalised
// keys and queries), but U = A (beta v) and the state carry the values' own
// magnitude, which may exceed the f16 range (65504).  The recurrence is linear
// in (v, S) jointly and the columns of S are independent, so the value path
// runs in powers of two: the WY stage stores U * 2^-uexp with uexp the
// smallest e >= 0 with max|beta v| * 2^-e <= kValueRange (one exponent per
// unit and channel pass), and every scan workgroup picks its own exponent for
// its columns (its chunks' uexp and its starting state), rescales U by the
// exact power of two and scales its outputs back on store.  With values below
// kValueRange (the common case) every exponent is 0 and nothing is rescaled.
struct WyBuffers {
  _Float16* W;
  _Float16* kgT;
  _Float16* U;
  float* decay;
  _Float16* qg;
  _Float16* Aqk;
  int32_t* uexp;
};

// Largest scaled |beta v| (and starting-state entry) the f16 value path
// admits: the state then stays below ~sqrt(K) * 2 * kValueRange < 2^14 at d <= 512.
constexpr float kValueRange = 256.f;

// exponent e >= 0 with m * 2^-e <= kValueRange (m >= 0; 0 for m = 0)
__device__ __forceinline__ int value_exponent(float m) {
  int x = 0;
  (void)frexpf(m, &x);  // m = f 2^x, f in [0.5, 1)
  const int e = x - 8;  // kValueRange = 2^8
  return e > 0 ? e : 0;
}

// 2^e for -126 <= e <= 127, built from the exponent bits (exact; with a
// uniform e the compiler keeps it in scalar registers)
__device__ __forceinline__ float pow2_exact(int e) { return __builtin_bit_cast(float, (127 + e) << 23); }

__host__ __device__ constexpr int wy_passes(int K) { return K > 256 ? K / 256 : 1; }

struct WyLayout {
  size_t off_W, off_kg, off_U, off_decay, off_qg, off_Aqk, off_uexp, total;
};

inline WyLayout wy_layout(int n_chunk, int H, int K, int V, bool causal) {
  const size_t units = (size_t)n_chunk * (size_t)H;
  WyLayout l{};
  size_t o = 0;
  l.off_W = o;     o = align256(o + units * kChunk * K * 2);
  l.off_kg = o;    o = align256(o + units * kChunk * K * 2);
  l.off_U = o;     o = align256(o + units * kChunk * V * 2);
  l.off_decay = o; o = align256(o + units * K * 4);
  l.off_qg = o;    if (causal) o = align256(o + units * kChunk * K * 2);
  l.off_Aqk = o;   if (causal) o = align256(o + units * kChunk * kChunk * 2);
  l.off_uexp = o;  o = align256(o + units * wy_passes(K) * 4);
  l.total = o;
  return l;
}

inline WyBuffers wy_buffers(void* ws, const WyLayout& l, bool causal) {
  char* base = (char*)ws;
  WyBuffers b;
  b.W = (_Float16*)(base + l.off_W);
  b.kgT = (_Float16*)(base + l.off_kg);
  b.U = (_Float16*)(base + l.off_U);
  b.decay = (float*)(base + l.off_decay);
  b.qg = causal ? (_Float16*)(base + l.off_qg) : nullptr;
  b.Aqk = causal ? (_Float16*)(base + l.off_Aqk) : nullptr;
  b.uexp = (int32_t*)(base + l.off_uexp);
  return b;
}

struct WyArgs {
  const __bf16* q;     // [T,H,K] (causal only)
  const __bf16* k;     // [T,H,K]
  const __bf16* v;     // [T,H,V]
  const float* g;      // [T,H,K] natural-log decay, or log2 cumsum when g_cumulative
  const void* beta;    // [T,H,V] f32 or bf16
  const __bf16* b;     // [T,H,K] or null
  const int32_t* chunk_tok0;
  const int32_t* chunk_len;
  int H;
  float scale;
  WyBuffers out;
  __bf16* A_ref;       // optional [T,H,64] bf16 inverse (reference layout)
  // raw projections (f_raw != null): q, k, v are then projection rows with the
  // strides below, g and beta come from f_raw / w_raw, b must be null
  const __bf16* f_raw;           // decay projection [T, f_stride]
  const __bf16* e_raw;           // erase logits [T, e_stride]
  const __bf16* w_raw;           // write logits [T, w_stride]
  const __bf16* decay_bias;      // [H*K]
  const __bf16* decay_scale_log; // [H]
  __bf16* q_hat;                 // [T,H,K] normalised q out, or null
  int64_t q_stride, k_stride, v_stride, f_stride, e_stride, w_stride;
  float eps;
};

// Two-level scan.  A sequence's chunks are split into groups of L chunks.
//   phase 1  per group (in parallel): the transition P_g = prod_c (Diag(decay_c) - kg_c^T W_c)
//            and the zero-start contribution Q_g, by running the scan on [I | 0]
//   phase 2  per sequence (serial over its groups): S_{g+1} = P_g S_g + Q_g
//   phase 3  per group (in parallel): the scan proper from S_g, with its outputs
// Sequence n owns the global groups [G_n, G_n + ceil(chunks_n / L)), G_n the
// running sum over earlier sequences; kernels locate their group from
// seq_chunk_offsets on the fly.
struct GroupBuffers {
  __bf16* P_hi;  // [n_group_bound, H, K, K] A-frag order (red = K), P_g = P_hi + P_lo
  __bf16* P_lo;
  float* Q;      // [n_group_bound, H, K, V] C-frag order (n = V)
  float* S0;     // [n_group_bound, H, K, V] C-frag order, state entering each group
};

// State columns one scan workgroup carries: all of them up to d = 128, and a
// 64-column slice at d = 256 and d = 512, so that the K x slice fp32 state and
// the prefetched chunk records fit the registers of two waves per SIMD (at
// d = 512 with a 60-byte spill; 32-column slices, without it, ran 12-16 %
// slower: twice the workgroups, each reading the head's full W and kg^T).
__host__ __device__ constexpr int scan_slice(int D) { return D > 128 ? 64 : D; }

// Chunks per group for the two-level scan (0 = plain per-sequence scan).
// The scan runs one workgroup per (sequence or group, head, column slice).
// Groups are used when the plain scan would occupy fewer than 256 workgroups
// (one per CU of the MI355X) and the sequences are long.  Sequence n has
// ceil(c_n / L) groups, and sum_n ceil(c_n / L) <= ceil(n_chunk / L) + n_seq - 1,
// so L = ceil(n_chunk / G) with G = 256 / (H slices) - (n_seq - 1) is the
// shortest group (at least 4 chunks) whose grid fits one round of 256
// workgroups: the scan's time is its longest group's.  (A 9 % longer second
// round, with power-of-two groups, cost the 4-segment 65536-token update a
// third more in the transition and scan kernels.)
// d = 512 always runs the plain scan: its group transition (K x K fp32 per
// head) does not fit the transition and combine kernels' register plans.
inline int scan_group_chunks(int n_chunk, int n_seq, int H, int V) {
  if (n_seq <= 0 || n_chunk <= 0 || V > 256) return 0;
  const long hs = (long)H * (V / scan_slice(V));
  if ((long)n_seq * hs >= 256) return 0;
  const long G = 256 / hs - (n_seq - 1);  // groups that fit a round
  if (G < 2) return 0;
  long L = ((long)n_chunk + G - 1) / G;
  if (L < 4) L = 4;
  if (n_chunk / n_seq < 2 * L) return 0;
  return (int)L;
}
inline int group_bound(int n_chunk, int n_seq, int L) { return n_chunk / L + n_seq + 1; }

inline size_t group_layout(size_t base, int n_chunk, int n_seq, int H, int K, int V, GroupBuffers* out,
                           void* ws) {
  const int L = scan_group_chunks(n_chunk, n_seq, H, V);
  if (L == 0) return base;
  const size_t nb = (size_t)group_bound(n_chunk, n_seq, L);
  size_t o = align256(base);
  const size_t off_Ph = o; o = align256(o + nb * H * K * K * 2);
  const size_t off_Pl = o; o = align256(o + nb * H * K * K * 2);
  const size_t off_Q = o; o = align256(o + nb * H * K * V * 4);
  const size_t off_S0 = o; o = align256(o + nb * H * K * V * 4);
  if (out != nullptr) {
    char* b = (char*)ws;
    out->P_hi = (__bf16*)(b + off_Ph);
    out->P_lo = (__bf16*)(b + off_Pl);
    out->Q = (float*)(b + off_Q);
    out->S0 = (float*)(b + off_S0);
  }
  return o;
}

// Where global group g of the two-level scan lies: sequence n owns the groups
// [G_n, G_n + cnt_n), cnt_n = ceil(chunks_n / L), G_n the sum over earlier
// sequences.  One wave scans the sequences 64 at a time; every lane returns
// the same values.
struct GroupLoc {
  int seq, c_begin, c_end, first_group, n_groups;
  bool valid;
};
__device__ __forceinline__ GroupLoc locate_group(const int32_t* soff, int n_seq, int L, int g) {
  const int lane = threadIdx.x & 63;
  int base = 0;
  for (int n0 = 0; n0 < n_seq; n0 += 64) {
    const int n = n0 + lane;
    int c0 = 0, c1 = 0, cnt = 0;
    if (n < n_seq) {
      c0 = soff[n];
      c1 = soff[n + 1];
      cnt = (c1 - c0 + L - 1) / L;
    }
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    const int first = base + incl - cnt;
    const unsigned long long hit = __ballot(n < n_seq && g >= first && g < first + cnt);
    if (hit != 0) {
      const int src = __ffsll((unsigned long long)hit) - 1;
      GroupLoc r;
      r.seq = n0 + src;
      r.first_group = __shfl(first, src, 64);
      r.n_groups = __shfl(cnt, src, 64);
      const int sc0 = __shfl(c0, src, 64), sc1 = __shfl(c1, src, 64);
      r.c_begin = sc0 + (g - r.first_group) * L;
      r.c_end = min(r.c_begin + L, sc1);
      r.valid = true;
      return r;
    }
    base += __shfl(incl, 63, 64);
  }
  GroupLoc r{};
  r.valid = false;
  return r;
}
struct StateArgs {
  WyBuffers in;
  const int32_t* chunk_tok0;
  const int32_t* chunk_len;
  const int32_t* seq_chunk_offsets;
  const int32_t* chunk_block_ids;
  const int32_t* chunk_flags;
  const float* h0;     // [N,H,K,V] or null; with h0_slot, [slots,H,K,V] indexed by h0_slot[seq]
  float* ht;           // [N,H,K,V] or null; with ht_slot, [slots,H,K,V] indexed by ht_slot[seq]
  const int32_t* h0_slot;  // [N] or null
  const int32_t* ht_slot;  // [N] or null
  float* snaps;        // [n_block,H,K,V] or null
  __bf16* o;           // [T,H,V] (causal output, or the fused snapshot read) or null
  // d <= 128, snapshot mode: the read o = bf16(scale * q_hat . bf16(rd_states[block]))
  // runs inside the scan when rd_states is set (never written by the same launch)
  const float* rd_states;  // [n_block,H,K,V] or null
  const __bf16* rd_q;      // q_hat [T,H,K]
  int H;
  int n_seq;
  int n_chunk;
  float scale;
  int group_L;         // chunks per group, 0 = plain scan
  GroupBuffers grp;    // valid when group_L > 0
};

// Gate and q/k prologue (models/qwen/layer.py:71-97).  Inputs are bf16 rows
// of H*D channels with a per-token stride in elements (views of the fused
// projection outputs); outputs are contiguous [rows = T*H, D].
struct PrologueArgs {
  const uint16_t* decay;            // f_down(decay latent) [T, stride]
  const uint16_t* decay_bias;       // [H*D]
  const uint16_t* decay_scale_log;  // [H]
  const uint16_t* erase;            // erase logits [T, stride]
  const uint16_t* write;            // write logits [T, stride]
  const uint16_t* q;                // raw q [T, stride] (QK only)
  const uint16_t* k;                // raw k [T, stride] (QK only)
  int64_t decay_stride, erase_stride, write_stride, q_stride, k_stride;
  float* g_out;                     // [T, H, D] fp32
  uint16_t* beta_out;               // [T, H, D] bf16
  uint16_t* erase_out;              // [T, H, D] bf16 sqrt(b) (gates only)
  uint16_t* q_out;                  // [T, H, D] bf16 (QK only)
  uint16_t* k_out;                  // [T, H, D] bf16 (QK only)
  int64_t rows;                     // T * H
  int H;
  float eps;
};

// Decode readout: one query row per sequence b; q and gate rows are
// `q_stride` / `gate_stride` elements apart (head h at offset h*K / h*V).
struct ReadoutArgs {
  const float* S;           // [slots, H, K, V] fp32
  const int32_t* slot_idx;  // [B] or null (slot = b)
  const __bf16* q;          // [B, q_stride] l2-normalised, or raw with MEMT_GDN2_READOUT_L2NORM_Q
  const __bf16* gate;       // [B, gate_stride]
  const __bf16* weight;     // [V]
  __bf16* out;              // [B, H*V]
  int64_t q_stride, gate_stride;
  int H;
  int flags;                // MEMT_GDN2_READOUT_* bits
  float scale, q_eps, eps, softcap;
  int gate_kind;
};

// Launchers (return hipError_t of the launch).
hipError_t launch_prologue(const PrologueArgs& a, int D, bool qk, hipStream_t stream);
hipError_t launch_wy(const WyArgs& a, int n_chunk, int K, int V, bool causal, bool g_cumulative,
                     bool beta_bf16, hipStream_t stream);
hipError_t launch_state(const StateArgs& a, int K, int V, bool causal, hipStream_t stream);
// d <= 128 column-split scan: phase 1 the group transitions (units = group bound),
// phase 0 the scan proper (units = groups, or sequences for the plain scan).
hipError_t launch_colscan(const StateArgs& a, int K, int V, bool causal, int phase, int units,
                          hipStream_t stream);
hipError_t launch_read_fwd(const __bf16* q, const float* snaps, __bf16* o, const int32_t* chunk_tok0,
                           const int32_t* chunk_len, const int32_t* chunk_block_ids, int n_chunk, int H,
                           int K, int V, float scale, hipStream_t stream, const int32_t* block_slot = nullptr);
hipError_t launch_readout(const ReadoutArgs& a, int B, int K, int V, bool state_bf16, hipStream_t stream);
hipError_t launch_rms_norm_gated(const __bf16* x, const __bf16* gate, const __bf16* weight, __bf16* out,
                                 int64_t rows, int dim, float eps, float softcap, int gate_kind,
                                 hipStream_t stream);
hipError_t launch_l2norm(const void* x, bool x_bf16, void* y, bool y_bf16, float* rstd, int64_t rows,
                         int dim, float eps, hipStream_t stream);
hipError_t launch_cumsum(const void* g, bool g_bf16, float* gk, const int32_t* chunk_tok0,
                         const int32_t* chunk_len, int n_chunk, int H, int S, float scale, bool reverse,
                         hipStream_t stream);
hipError_t launch_wy_export(const WyBuffers& in, const int32_t* chunk_tok0, const int32_t* chunk_len,
                            int n_chunk, int H, int K, int V, __bf16* w, __bf16* u, __bf16* kg,
                            __bf16* Aqk, __bf16* qg, hipStream_t stream);
hipError_t launch_wy_import(const __bf16* w, const __bf16* u, const __bf16* kg, const float* gk,
                            const int32_t* chunk_tok0, const int32_t* chunk_len, int n_chunk, int H,
                            int K, int V, WyBuffers out, hipStream_t stream);

}  // namespace memt
