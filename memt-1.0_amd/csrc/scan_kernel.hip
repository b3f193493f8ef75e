// Column-split state scan of the chunked GDN-2 update for d <= 128 (K == V).
//
// Same recurrence as state_kernel.hip (models/qwen/ops/_triton/state.py:76-115):
//   snapshot S if the chunk starts a read block
//   V_new = U - W . f16(S)
//   o     = scale * qg . f16(S) + Aqk . V_new        (causal output)
//   S     = decay * S + kg^T . f16(V_new)            (if committed)
// with a different division of the work.  Each wave owns V/4 state columns
// over all K rows, so every product of a chunk chains through its own
// registers: the C fragments of S are, element for element, the f16 B (and
// A) operands of the next product under the P-frag reduction order, and the C
// fragments of V_new are the operands of the state update and of the output.
// No operand crosses waves through LDS and the chunk has no barrier of its own.
//
// What the waves share are the chunk records (W, kg^T, qg, Aqk and the decay
// row), read by every wave in full.  They are staged in LDS by direct
// global-to-LDS loads (16 bytes per lane, one 1 KiB operand fragment per
// instruction), double-buffered: while chunk c computes from one buffer the
// records of chunk c + 1 land in the other, and one barrier per chunk (after
// the loads have landed and every wave is done with the buffer) hands them over.
// U, of which each wave reads only its own columns, comes through the same
// buffers, so the chunk loop has no global load into registers to wait for.
//
// In snapshot mode (every token reads the state its read block starts from,
// read_states[block], not the evolving S) the read runs here too when the
// launch writes no read state: each chunk's q_hat rows ride in the record
// buffers (16-byte slots at a pitch of K / 8 + 1 slots, so the rows of an
// operand read fall on distinct LDS banks), each wave holds bf16 of its columns
// of the read state as MFMA operands, and o^T = bf16(S_read)^T q_hat^T is one
// bf16 MFMA product per chunk with read_fwd_kernel's operand slots and step
// order, so o is that kernel's output bit for bit.  It replaces a separate pass
// that read q_hat and the state tile again.
//
// Kernels:
//   colscan_state_kernel  4 waves per (sequence or group, head): the scan with
//                         its outputs (o, snapshots, ht)
//   colscan_trans_kernel  8 waves per (group, head): waves 0-3 carry the columns
//                         of the group transition P_g (from the identity, no
//                         values), waves 4-7 those of Q_g (from zero, with U);
//                         both read the same W / kg^T records from LDS.
// The combine between them is state_kernel.hip's combine_kernel, unchanged.
#include "gdn2_internal.h"

namespace memt {
namespace {

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef const __attribute__((address_space(3))) char lds_cchar;
constexpr int kFrag = 1024;  // bytes of one operand fragment: 64 lanes x 16 B

// LDS reads at a per-lane base plus a compile-time byte offset (the offset
// folds into the instruction's immediate)
__device__ __forceinline__ f16x8 lds_f16x8(lds_cchar* base, int off) {
  return *(const __attribute__((address_space(3))) f16x8*)(base + off);
}
__device__ __forceinline__ f32x4 lds_f32x4(lds_cchar* base, int off) {
  return *(const __attribute__((address_space(3))) f32x4*)(base + off);
}

// One direct load: lane l's 16 bytes at src_lane land at dst + 16 l (dst is
// uniform over the wave and 16-byte aligned).
__device__ __forceinline__ void dma16(const void* src_lane, char* dst) {
  __builtin_amdgcn_global_load_lds(src_lane, (lds_ptr)dst, 16, 0, 0);
}
// every outstanding global access of the wave (the direct loads included) done,
// then the workgroup barrier
__device__ __forceinline__ void vm_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }


// LDS buffer of one chunk's records, in fragments of 1 KiB: W, kg^T, (qg and
// Aqk for the causal output), U and the decay row.  Every record but the decay
// row spans a multiple of NW fragments, so the record a wave's i-th load belongs
// to is known at compile time; the decay row (K floats) takes one slot, loaded
// by wave 0.  U comes through LDS too although each wave reads only its own
// columns of it: with no global load into registers in the chunk loop, the
// compiler has nothing to wait for there, and the chunk's only wait is the
// explicit one before its barrier.
// RD: the snapshot read runs inside the scan, and the buffer also holds the
// chunk's q_hat rows after the decay row, in 16-byte slots at a pitch of K / 8 + 1
// slots per row (the spare slot puts the 16 rows an operand read touches on
// distinct LDS banks), in whole rounds of the NW waves' direct loads.
template <int K, bool CAUSAL, bool TRANS, bool RD = false>
struct RecordBuf {
  static constexpr int NW = TRANS ? 8 : 4;
  static constexpr int NFW = K / 8;  // fragments of a 64 x K (or 64 x V, K == V) f16 record
  static_assert(NFW % NW == 0 && 8 % 4 == 0, "records in whole rounds of waves");
  static constexpr bool OUT = CAUSAL && !TRANS;
  static constexpr int F_W = 0, F_KG = NFW;
  static constexpr int F_QG = 2 * NFW;
  static constexpr int F_AQ = F_QG + (OUT ? NFW : 0);
  static constexpr int F_U = F_AQ + (OUT ? 8 : 0);
  static constexpr int F_D = F_U + NFW;
  static constexpr int QSPR = K / 8 + 1;  // slots of one q_hat row
  static constexpr int F_Q = F_D + 1;
  static constexpr int NFQ = RD ? (kChunk * QSPR + 64 * NW - 1) / (64 * NW) * NW : 0;
  static constexpr int NF = F_Q + NFQ;
  static constexpr int BYTES = NF * kFrag;
};

// Issue the direct loads of chunk unit u's records into buf: round i of the
// NW waves loads fragments NW i .. NW i + NW - 1, wave w the (NW i + w)-th.
template <int K, bool CAUSAL, bool TRANS, bool RD = false>
__device__ __forceinline__ void stage_records(const WyBuffers& in, size_t u, char* buf, int w, int lane) {
  using B = RecordBuf<K, CAUSAL, TRANS, RD>;
  constexpr int NW = B::NW;
#pragma unroll
  for (int i = 0; i < B::F_D / NW; ++i) {
    const int f0 = NW * i;  // compile time: which record
    const char* src;
    if (f0 < B::F_KG) {
      src = (const char*)in.W + (u * B::NFW + f0 + w) * kFrag;
    } else if (f0 < B::F_QG) {
      src = (const char*)in.kgT + (u * B::NFW + (f0 - B::F_KG) + w) * kFrag;
    } else if (B::OUT && f0 < B::F_AQ) {
      src = (const char*)in.qg + (u * B::NFW + (f0 - B::F_QG) + w) * kFrag;
    } else if (B::OUT && f0 < B::F_U) {
      src = (const char*)in.Aqk + (u * 8 + (f0 - B::F_AQ) + w) * kFrag;
    } else {
      src = (const char*)in.U + (u * B::NFW + (f0 - B::F_U) + w) * kFrag;
    }
    dma16(src + 16 * lane, buf + (f0 + w) * kFrag);
  }
  // K / 4 pieces of 16 bytes; lanes past them repeat the row
  if (w == 0) dma16((const char*)(in.decay + u * K) + 16 * (lane % (K / 4)), buf + B::F_D * kFrag);
}

// Role of a wave: 0 the scan proper, 1 the columns of P_g, 2 those of Q_g.
template <int K, int V, bool CAUSAL, bool TRANS, bool RD = false>
__device__ __forceinline__ void colscan(const StateArgs& a, int unitg, int h, char* lds) {
  static_assert(K == V && (K == 64 || K == 128), "column-split scan: K == V <= 128");
  static_assert(!RD || (!CAUSAL && !TRANS), "the fused read is the snapshot mode's");
  using B = RecordBuf<K, CAUSAL, TRANS, RD>;
  constexpr bool OUT = B::OUT;
  constexpr int CW = V / 4, CT = CW / 16;  // columns and 16-column tiles per wave
  constexpr int KS = K / 32, RT = K / 16;  // channel steps, 16-row tiles of the state
  constexpr int TQ = kChunk / 16;          // token tiles of a chunk
  const int H = a.H;

  int c_begin, c_end, seq = unitg;
  bool first = true, last = true;
  if (a.group_L == 0) {
    c_begin = a.seq_chunk_offsets[seq];
    c_end = a.seq_chunk_offsets[seq + 1];
  } else {
    const GroupLoc gl = locate_group(a.seq_chunk_offsets, a.n_seq, a.group_L, unitg);
    if (!gl.valid) return;
    seq = __builtin_amdgcn_readfirstlane(gl.seq);
    c_begin = __builtin_amdgcn_readfirstlane(gl.c_begin);
    c_end = __builtin_amdgcn_readfirstlane(gl.c_end);
    const int g_first = __builtin_amdgcn_readfirstlane(gl.first_group);
    const int g_count = __builtin_amdgcn_readfirstlane(gl.n_groups);
    first = unitg == g_first;
    last = unitg + 1 == g_first + g_count;
    if (TRANS && last) return;  // the last group's transition is never used
  }

  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int role = TRANS ? 1 + (w >> 2) : 0;  // uniform over the wave
  const int col0 = CW * (w & 3);               // first state column of this wave

  // ---- prologue: everything the first chunk needs is requested at once ----
  int mbase = c_begin - 64;
  int m_flags = 0, m_uexp = 0, m_block = -1, m_tok0 = 0, m_len = 0;
  int flags = 0, block = -1, tok0 = 0, len = 0;
  // plan entries of chunks [mbase, mbase + 64), one chunk per lane, read with
  // readlane; the chunk's U exponent joins bits 8.. of the flags there (not at
  // the load, which would make the prologue wait for these loads right after
  // issuing the first chunk's direct loads)
  auto meta_load = [&](int c) {
    mbase = c;
    const int cc = c + lane;
    const bool ok = cc < c_end;
    m_flags = !ok ? 0 : a.chunk_flags ? a.chunk_flags[cc] : MEMT_GDN2_CHUNK_COMMIT;
    m_uexp = ok ? a.in.uexp[(size_t)cc * H + h] : 0;
    if constexpr (!TRANS) {
      m_block = (ok && (RD || a.snaps != nullptr) && a.chunk_block_ids != nullptr) ? a.chunk_block_ids[cc] : -1;
      if constexpr (CAUSAL || RD) {
        m_tok0 = ok ? a.chunk_tok0[cc] : 0;
        m_len = ok ? a.chunk_len[cc] : 0;
      }
    }
  };
  auto meta = [&](int c) {
    if (c - mbase >= 64) {
      meta_load(c);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    const int i = c - mbase;
    flags = __builtin_amdgcn_readlane(m_flags, i) | (__builtin_amdgcn_readlane(m_uexp, i) << 8);
    block = __builtin_amdgcn_readlane(m_block, i);
    tok0 = (CAUSAL || RD) ? __builtin_amdgcn_readlane(m_tok0, i) : 0;
    len = (CAUSAL || RD) ? __builtin_amdgcn_readlane(m_len, i) : 0;
  };
  // RD: chunk c2's q_hat rows into buffer bf by direct loads.  Slot g = 64 f + lane
  // of fragment f holds piece g % QSPR of row g / QSPR (the spare piece repeats the
  // row's first; rows past the chunk, and past the tile, repeat its last row).
  auto stage_q = [&](int c2, char* bf) {
    if constexpr (RD) {
      int t0, ln;
      if (c2 - mbase < 64) {
        t0 = __builtin_amdgcn_readlane(m_tok0, c2 - mbase);
        ln = __builtin_amdgcn_readlane(m_len, c2 - mbase);
      } else {
        t0 = a.chunk_tok0[c2];
        ln = a.chunk_len[c2];
      }
      const __bf16* qh = a.rd_q + (size_t)h * K;
#pragma unroll
      for (int i = 0; i < B::NFQ / B::NW; ++i) {
        const int f = B::NW * i + w, sg = 64 * f + lane;
        const int row = min(sg / B::QSPR, ln - 1), piece = sg % B::QSPR;
        dma16(qh + (size_t)(t0 + row) * H * K + 8 * (piece < K / 8 ? piece : 0), bf + (B::F_Q + f) * kFrag);
      }
    }
  };

  // two record buffers: chunk c computes from one while chunk c + 1's records
  // land in the other (a third, with two chunks in flight, measured slower in
  // the transition kernel: 29.5 -> 32.7 us at 16 heads, 8192 tokens, d = 128)
  constexpr int NBUF = 2;
  auto buf = [&](int r) { return lds + (r % NBUF) * B::BYTES; };
  // RD: bf16 of the read state, the A operand of o^T = bf16(S_read)^T q_hat^T:
  // element j of (s, ct) is S_read[32 s + 8 lg + j][col0 + 16 ct + lr]
  bf16x8 sr[RD ? KS : 1][RD ? CT : 1];
  int sr_block = -1;
  auto load_sr = [&](int blk) {
    if constexpr (RD) {
      const float* sp = a.rd_states + ((size_t)blk * H + h) * K * V + col0 + lr;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int j = 0; j < 8; ++j) sr[s][ct][j] = (__bf16)sp[(size_t)(32 * s + 8 * lg + j) * V + 16 * ct];
      sr_block = blk;
    }
  };
  if (c_begin < c_end) {
    meta_load(c_begin);
#pragma unroll
    for (int j = 0; j < NBUF - 1; ++j)
      if (c_begin + j < c_end) {
        stage_records<K, CAUSAL, TRANS, RD>(a.in, (size_t)(c_begin + j) * H + h, buf(j), w, lane);
        stage_q(c_begin + j, buf(j));
      }
    if constexpr (RD) load_sr(__builtin_amdgcn_readfirstlane(a.chunk_block_ids[c_begin]));
  }

  // the starting state, tile (rt, ct): rows 16 rt + 4 lg + e, column col0 + 16 ct + lr.
  // Every group of a multi-group sequence starts from the combine's S0 (the first
  // one from the combine's copy of h0), so when ht and h0 name the same slot the
  // last group's ht write cannot overtake the first group's h0 read.
  const bool from_s0 = !TRANS && !(first && last);
  const int slot = (!from_s0 && a.h0_slot) ? a.h0_slot[seq] : seq;
  const float* h0p = (!TRANS && a.h0 != nullptr) ? a.h0 + ((size_t)slot * H + h) * K * V : nullptr;
  const float* s0p = a.grp.S0 + ((size_t)unitg * H + h) * K * V;
  f32x4 S[RT][CT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      if (from_s0) {
        S[rt][ct] = *(const f32x4*)(s0p + ((size_t)(rt * (V / 16) + (col0 >> 4) + ct) * 64 + lane) * 4);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * rt + 4 * lg + e, col = col0 + 16 * ct + lr;
          S[rt][ct][e] = role == 1 ? (row == col ? 1.f : 0.f)
                                   : h0p ? h0p[4 * lg * V + col0 + lr + (16 * rt + e) * V + 16 * ct] : 0.f;
        }
      }
    }
  // Value exponent of this wave's columns: the largest of its chunks' U exponents
  // and of its starting state's, so that U 2^-ew and S 2^-ew stay inside the f16
  // operand range.  Columns of S are independent, so each wave has its own; the
  // transition (role 1) is scale-free.
  int ew = 0;
  if (role != 1) {
    int eu = 0;
    for (int c0 = c_begin; c0 < c_end; c0 += 64) {
      const int c = c0 + lane;
      if (c < c_end) eu = max(eu, a.in.uexp[(size_t)c * H + h]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) eu = max(eu, __shfl_xor(eu, off, 64));
    float smax = 0.f;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) smax = fmaxf(smax, fabsf(S[rt][ct][e]));
    ew = __builtin_amdgcn_readfirstlane(max(eu, value_exponent(wave_max(smax))));
  }
  const float oscale = pow2_exact(ew);  // back to the values' own scale on store
  const float iscale = pow2_exact(-ew);
  if (role != 1) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) S[rt][ct] *= iscale;
  }
  vm_barrier();  // the first chunk's records are in LDS

  for (int c = c_begin; c < c_end; ++c) {
    const int r = c - c_begin, b = r % NBUF;
    // this lane's view of the chunk's buffer: fragment f is at + f * kFrag
    lds_cchar* const cur = (lds_cchar*)lds + b * B::BYTES + 16 * lane;
    meta(c);
    const int cur_flags = flags, cur_tok0 = tok0, cur_len = len, cur_block = block;
    // the next chunk's shared records into the other buffer
    const bool ahead = c + NBUF - 1 < c_end;  // the records NBUF - 1 chunks ahead into the free buffer
    if (ahead) {
      stage_records<K, CAUSAL, TRANS, RD>(a.in, (size_t)(c + NBUF - 1) * H + h, buf(r + NBUF - 1), w, lane);
      stage_q(c + NBUF - 1, buf(r + NBUF - 1));
    }
    if constexpr (RD) {
      if (cur_block != sr_block) load_sr(cur_block);  // a read block that starts inside the range
    }
    if constexpr (!TRANS) {
      if (a.snaps != nullptr && cur_block >= 0 && (cur_flags & MEMT_GDN2_CHUNK_BLOCK_START)) {
        // one per-lane pointer and constant offsets, so no per-element address
        // stays live across the loop
        float* sn = a.snaps + ((size_t)cur_block * H + h) * K * V + 4 * lg * V + col0 + lr;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e) sn[(16 * rt + e) * V + 16 * ct] = S[rt][ct][e] * oscale;
      }
    }
    auto frag = [&](int f) { return lds_f16x8(cur, f * kFrag); };

    // f16(S) operands of channel step s: slot j is row 32 s + 16 (j / 4) + 4 lg + j % 4
    auto s_operand = [&](int s, int ct) {
      f16x8 r;
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] = (_Float16)S[2 * s + (j >> 2)][ct][j & 3];
      return r;
    };
    // A product over the channel steps with the record fragments of step s + 1
    // read while step s multiplies; the scheduling barriers keep the compiler from
    // hoisting every read of the chunk at once.
    auto channel_product = [&](int f_base, f32x4 (&out)[TQ][CT], bool s_is_a) {
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) out[tq][ct] = zero4();
      f16x8 rf[2][TQ];
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq) rf[0][tq] = frag(f_base + tq * KS);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        if (s + 1 < KS) {
#pragma unroll
          for (int tq = 0; tq < TQ; ++tq) rf[(s + 1) & 1][tq] = frag(f_base + tq * KS + s + 1);
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const f16x8 sb = s_operand(s, ct);
#pragma unroll
          for (int tq = 0; tq < TQ; ++tq)
            out[tq][ct] = s_is_a ? mfma_f16(sb, rf[s & 1][tq], out[tq][ct]) : mfma_f16(rf[s & 1][tq], sb, out[tq][ct]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    // ---- V_new = U 2^(uexp - ew) - W f16(S) ----
    f16x8 Vb[2][CT];  // f16(V_new) operands: slot j of token step s2 is token 32 s2 + 16 (j / 4) + 4 lg + j % 4
    {
      // this wave's columns of U (C fragments, 8 bytes per lane and tile)
      f16x4 uf[TQ][CT];
      lds_cchar* const ub = (lds_cchar*)lds + b * B::BYTES + B::F_U * kFrag + 8 * lane + (col0 >> 4) * 512;
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          uf[tq][ct] = *(const __attribute__((address_space(3))) f16x4*)(ub + (tq * (V / 16) + ct) * 512);
      f32x4 acc[TQ][CT];
      channel_product(B::F_W, acc, false);
      const float uscale = pow2_exact((cur_flags >> 8) - ew);  // <= 1
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float u = role == 1 ? 0.f : (float)uf[tq][ct][e] * uscale;
            Vb[tq >> 1][ct][4 * (tq & 1) + e] = (_Float16)(u - acc[tq][ct][e]);
          }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (OUT) {
      // o^T = f16(S)^T qg^T (tile [ct][tq] kept as [tq][ct]), then scale and
      // + f16(V_new)^T Aqk^T; lane holds o[16 tq + lr][col0 + 16 ct + 4 lg + e]
      f32x4 acco[TQ][CT];
      channel_product(B::F_QG, acco, true);
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq) {
        const f16x8 af0 = frag(B::F_AQ + tq * 2), af1 = frag(B::F_AQ + tq * 2 + 1);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          acco[tq][ct] *= a.scale;
          acco[tq][ct] = mfma_f16(Vb[0][ct], af0, acco[tq][ct]);
          acco[tq][ct] = mfma_f16(Vb[1][ct], af1, acco[tq][ct]);
        }
        const int t = 16 * tq + lr;
        if (t < cur_len) {
          __bf16* orow = a.o + ((size_t)(cur_tok0 + t) * H + h) * V + col0 + 4 * lg;
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            bf16x4 o4;
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = (__bf16)(acco[tq][ct][e] * oscale);
            *(bf16x4*)(orow + 16 * ct) = o4;
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (RD) {
      // ---- the snapshot read: o^T = bf16(S_read)^T q_hat^T, lane holds
      // o[16 tq + lr][col0 + 16 ct + 4 lg + e]; the operands' slots and the order
      // over the channel steps are read_fwd_kernel's, so the values are its bits
      lds_cchar* const qb = (lds_cchar*)lds + b * B::BYTES + B::F_Q * kFrag + (lr * B::QSPR + lg) * 16;
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq) {
        f32x4 acc[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[ct] = zero4();
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const bf16x8 qv = *(const __attribute__((address_space(3))) bf16x8*)(qb + (16 * tq * B::QSPR + 4 * s) * 16);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) acc[ct] = mfma_bf16(sr[s][ct], qv, acc[ct]);
        }
        const int t = 16 * tq + lr;
        if (t < cur_len) {
          __bf16* orow = a.o + ((size_t)(cur_tok0 + t) * H + h) * V + col0 + 4 * lg;
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            bf16x4 o4;
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = (__bf16)(acc[ct][e] * a.scale);
            *(bf16x4*)(orow + 16 * ct) = o4;
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // ---- S = decay S + kg^T f16(V_new), by 16-row tile ----
    if (cur_flags & MEMT_GDN2_CHUNK_COMMIT) {
      f16x8 kf[2][2];
      f32x4 dv[2];
      auto read_tile = [&](int rt, int slot) {
        kf[slot][0] = frag(B::F_KG + rt * 2);
        kf[slot][1] = frag(B::F_KG + rt * 2 + 1);
        dv[slot] = lds_f32x4(cur - 16 * lane + 16 * lg, B::F_D * kFrag + 64 * rt);  // rows 16 rt + 4 lg ..
      };
      read_tile(0, 0);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        if (rt + 1 < RT) read_tile(rt + 1, (rt + 1) & 1);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          S[rt][ct] *= dv[rt & 1];
          S[rt][ct] = mfma_f16(kf[rt & 1][0], Vb[0][ct], S[rt][ct]);
          S[rt][ct] = mfma_f16(kf[rt & 1][1], Vb[1][ct], S[rt][ct]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    vm_barrier();  // next chunk's records landed; every wave is done with this buffer
  }

  if constexpr (TRANS) {
    if (role == 2) {
      float* qo = a.grp.Q + ((size_t)unitg * H + h) * K * V;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          *(f32x4*)(qo + ((size_t)(rt * (V / 16) + (col0 >> 4) + ct) * 64 + lane) * 4) = S[rt][ct] * oscale;
    } else {
      // P_g row-major into LDS (the record buffers are dead), then read back by rows
      constexpr int PP = K + 4;
      float* pl = (float*)lds;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e) pl[(16 * rt + 4 * lg + e) * PP + col0 + 16 * ct + lr] = S[rt][ct][e];
    }
    __syncthreads();
    if (role == 1) {
      // split bf16 hi + lo in A-frag order (rows = P rows, reduction = P columns):
      // item i covers P[16 rt + l % 16][32 s + 8 (l / 16) + 0..7], l = i % 64
      constexpr int PP = K + 4;
      const float* pl = (const float*)lds;
      const size_t base = ((size_t)unitg * H + h) * K * K;
      const int t4 = tid;  // 0 .. 255 over the four P waves
#pragma unroll
      for (int i0 = 0; i0 < K * K / 8; i0 += 256) {
        const int i = i0 + t4, l = i & 63, rs = i >> 6;
        const int row = 16 * (rs / KS) + (l & 15), col = 32 * (rs % KS) + 8 * (l >> 4);
        const f32x4 x0 = *(const f32x4*)(pl + row * PP + col);
        const f32x4 x1 = *(const f32x4*)(pl + row * PP + col + 4);
        bf16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = e < 4 ? x0[e] : x1[e - 4];
          hi[e] = (__bf16)x;
          lo[e] = (__bf16)(x - (float)hi[e]);
        }
        *(bf16x8*)(a.grp.P_hi + base + (size_t)i * 8) = hi;
        *(bf16x8*)(a.grp.P_lo + base + (size_t)i * 8) = lo;
      }
    }
  } else if (last && a.ht != nullptr) {
    float* out = a.ht + ((size_t)(a.ht_slot ? a.ht_slot[seq] : seq) * H + h) * K * V;
    float* outl = out + 4 * lg * V + col0 + lr;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) outl[(16 * rt + e) * V + 16 * ct] = S[rt][ct][e] * oscale;
  }
}

template <int K, bool CAUSAL, bool TRANS, bool RD = false>
constexpr int colscan_lds() {
  constexpr int rec = 2 * RecordBuf<K, CAUSAL, TRANS, RD>::BYTES;
  constexpr int pst = TRANS ? K * (K + 4) * 4 : 0;
  return rec > pst ? rec : pst;
}

// One workgroup per (sequence or group, head): blocks b = unit * H + head.
template <int K, int V, bool CAUSAL, bool RD = false>
__global__ __launch_bounds__(256) void colscan_state_kernel(StateArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[colscan_lds<K, CAUSAL, false, RD>()];
  colscan<K, V, CAUSAL, false, RD>(a, blockIdx.x / a.H, blockIdx.x % a.H, lds);
}

template <int K, int V>
__global__ __launch_bounds__(512) void colscan_trans_kernel(StateArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[colscan_lds<K, false, true>()];
  colscan<K, V, false, true>(a, blockIdx.x / a.H, blockIdx.x % a.H, lds);
}

}  // namespace

hipError_t launch_colscan(const StateArgs& a, int K, int V, bool causal, int phase, int units, hipStream_t stream) {
  const dim3 grid(units * a.H);
  if (K == 128 && V == 128) {
    if (phase == 1) hipLaunchKernelGGL((colscan_trans_kernel<128, 128>), grid, dim3(512), 0, stream, a);
    else if (causal) hipLaunchKernelGGL((colscan_state_kernel<128, 128, true>), grid, dim3(256), 0, stream, a);
    else if (a.rd_states) hipLaunchKernelGGL((colscan_state_kernel<128, 128, false, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((colscan_state_kernel<128, 128, false>), grid, dim3(256), 0, stream, a);
  } else if (K == 64 && V == 64) {
    if (phase == 1) hipLaunchKernelGGL((colscan_trans_kernel<64, 64>), grid, dim3(512), 0, stream, a);
    else if (causal) hipLaunchKernelGGL((colscan_state_kernel<64, 64, true>), grid, dim3(256), 0, stream, a);
    else if (a.rd_states) hipLaunchKernelGGL((colscan_state_kernel<64, 64, false, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((colscan_state_kernel<64, 64, false>), grid, dim3(256), 0, stream, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace memt
