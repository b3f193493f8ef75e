// Readout, normalisation and layout kernels of the GDN-2 memory path.
#include "gdn2_internal.h"

#include <algorithm>
#include <atomic>

namespace memt {
namespace {

// ---------------------------------------------------------------------------
// Snapshot reader (models/qwen/ops/_triton/read.py:22-71) for d = 64: per
// (chunk, head), o[t] = bf16(scale * q[t] . bf16(S_block)), bf16 MFMA, fp32
// accumulation.  A workgroup takes all V state columns of one head for a run of
// kReadRun consecutive chunks, and reloads the bf16 state tile only when the
// block changes.  Wave w handles token rows [16w, 16w + 16); it issues all of a
// chunk's q loads before its first product, so a chunk costs one memory
// latency rather than one per 32 channels.
// ---------------------------------------------------------------------------
// chunks per reader workgroup (snapshot mode at 16 heads, 8192 tokens, d = 128:
// runs of 1, 2, 8 or 16 chunks measured 2-17 % slower than 4)
constexpr int kReadRun = 4;
constexpr int kWideCols = 128;  // state columns per read_wide_kernel workgroup (heads this wide read there)

template <int K, int V>
__global__ __launch_bounds__(256) void read_fwd_kernel(const __bf16* __restrict__ q,
                                                       const float* __restrict__ snaps,
                                                       __bf16* __restrict__ o, const int32_t* chunk_tok0,
                                                       const int32_t* chunk_len, const int32_t* block_ids,
                                                       int n_chunk, int n_units, int H, float scale,
                                                       const int32_t* block_slot) {
  constexpr int CB = V, SKP = K + 8, per = kReadRun;
  static_assert(V < kWideCols, "d >= 128 reads in read_wide_kernel");
  __shared__ __attribute__((aligned(16))) __bf16 S_lds[CB * SKP];  // column-major bf16(S)
  const int unit = blockIdx.x;  // (run, head)
  if (unit >= n_units) return;
  const int h = unit % H, col0 = 0;
  const int c_begin = (unit / H) * per, c_end = min(c_begin + per, n_chunk);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  int loaded = -1;
  for (int chunk = c_begin; chunk < c_end; ++chunk) {
    const int tok0 = chunk_tok0[chunk], len = chunk_len[chunk];
    const int blk = block_ids[chunk];
    if (blk != loaded) {
      if (loaded >= 0) __syncthreads();  // every wave is done with the previous tile
      // NL 16-byte loads per thread, issued in batches of up to 8 ahead of
      // their conversions, so a batch costs one memory latency
      const float* Sp = snaps + ((size_t)(block_slot ? block_slot[blk] : blk) * H + h) * K * V + col0;
      constexpr int NL = K * CB / 4 / 256, BATCH = NL < 8 ? NL : 8;
      static_assert(NL * 256 * 4 == K * CB && NL % BATCH == 0, "state tile split");
#pragma unroll 1
      for (int j0 = 0; j0 < NL; j0 += BATCH) {
        f32x4 s4[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
          const int idx = tid + 256 * (j0 + j);
          s4[j] = *(const f32x4*)(Sp + (size_t)(idx / (CB / 4)) * V + (idx % (CB / 4)) * 4);
        }
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
          const int idx = tid + 256 * (j0 + j);
          const int row = idx / (CB / 4), c4 = (idx % (CB / 4)) * 4;
#pragma unroll
          for (int e = 0; e < 4; ++e) S_lds[(c4 + e) * SKP + row] = (__bf16)s4[j][e];
        }
      }
      __syncthreads();
      loaded = blk;
    }
    // All K/32 q operands of this lane's row are loaded before the first
    // product, so the chunk pays one memory latency.  Rows past the chunk end
    // read its last row (they feed only output rows that are not stored); an
    // empty chunk loads nothing.
    const int t = 16 * w + lr;
    bf16x8 qa[K / 32];
    if (len > 0) {
      const __bf16* qp = q + ((size_t)(tok0 + min(t, len - 1)) * H + h) * K + 8 * lg;
#pragma unroll
      for (int s = 0; s < K / 32; ++s) qa[s] = *(const bf16x8*)(qp + 32 * s);
    } else {
#pragma unroll
      for (int s = 0; s < K / 32; ++s) qa[s] = bf16x8{};
    }
    f32x4 acc[CB / 16];
#pragma unroll
    for (int ct = 0; ct < CB / 16; ++ct) acc[ct] = zero4();
#pragma unroll
    for (int s = 0; s < K / 32; ++s) {
#pragma unroll
      for (int ct = 0; ct < CB / 16; ++ct) {
        const bf16x8 sb = *(const bf16x8*)(&S_lds[(16 * ct + lr) * SKP + 32 * s + 8 * lg]);
        acc[ct] = mfma_bf16(qa[s], sb, acc[ct]);
      }
    }
#pragma unroll
    for (int ct = 0; ct < CB / 16; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tt = 16 * w + 4 * lg + e;
        if (tt < len) o[((size_t)(tok0 + tt) * H + h) * V + col0 + 16 * ct + lr] = (__bf16)(acc[ct][e] * scale);
      }
  }
}

// ---------------------------------------------------------------------------
// Snapshot reader for d = 128, 256 and 512: read_fwd_kernel's product with the
// state held in registers.  A workgroup takes 128 state columns of one head for
// a run of chunks, 4 waves of 32 columns (each q operand read from LDS feeds two
// products).  Each wave holds its columns of bf16(S), all K channels (128
// registers at d = 512), as the A
// operand of o^T = bf16(S)^T q^T, loaded once per block, so the state is
// read from memory once per run instead of from LDS for every 16 tokens.  The
// q rows come through LDS by direct loads in steps of a chunk (half a chunk at
// d = 512, so that two workgroups share a CU and one covers the other's waits),
// double-buffered: step i + 1's rows land while step i is multiplied.  The
// operand slots and the order of the products over the channels are
// read_fwd_kernel's, so the output is bit-identical to it.  The NH workgroups of
// one (run, head) read the same q rows; their block indices are 8 apart, so they
// share an XCD and its L2 (HBM fetches at d = 512: q and the state once).
// ---------------------------------------------------------------------------
// rows of q per step: half a chunk at d = 512, so that two workgroups fit a CU's LDS
__host__ __device__ constexpr int wide_rows(int K) { return K > 256 ? 32 : kChunk; }
// waves per workgroup: four of 32 columns, two product tiles per q operand read
// from LDS (128 registers of state at d = 512).  Against eight waves of 16 columns:
// 0.42 -> 0.37 ms at d = 512 (64 heads, 8192 tokens), 0.30 -> 0.23 ms at d = 256
// (64 heads, 16384 tokens), 19.5 -> 16.3 us at d = 128 (16 heads, 8192 tokens)
constexpr int kWideWaves = 4;
// workgroups per CU: two at d >= 256 (66 KB of LDS each), four at d = 128 (34 KB)
__host__ __device__ constexpr int wide_per_cu(int K) { return K > 128 ? 2 : 4; }
template <int K>
struct WideReadLds {
  static constexpr int TS = wide_rows(K);                        // token rows per step
  static constexpr int QSPR = K / 8 + 1;                         // 16-byte slots per q row: K / 8 and a spare
  static constexpr int NF = (TS * QSPR * 16 + 1023) / 1024;      // direct loads (1 KiB each) per step
  static constexpr int BYTES = NF * 1024;                        // one step's buffer
  static constexpr int PIECE = 32 * kWideCols * 4;               // 32 state rows of the workgroup's columns, fp32
  static constexpr int NSLOT = BYTES / PIECE;                    // state pieces a buffer holds
};

// s_waitcnt vmcnt(N) (N a constant), then the workgroup barrier
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <int K, int V>
__global__ __launch_bounds__(64 * kWideWaves, kWideWaves * wide_per_cu(K) / 4) void read_wide_kernel(const __bf16* __restrict__ q,
                                                        const float* __restrict__ snaps,
                                                        __bf16* __restrict__ o,
                                                        const int32_t* __restrict__ chunk_tok0,
                                                        const int32_t* __restrict__ chunk_len,
                                                        const int32_t* __restrict__ block_ids, int n_chunk,
                                                        int n_units, int per, int H, float scale,
                                                        const int32_t* __restrict__ block_slot) {
  using L = WideReadLds<K>;
  constexpr int NW = kWideWaves, CWN = kWideCols / (16 * NW);  // waves, 16-column tiles per wave
  constexpr int NH = V / kWideCols, KS = K / 32, QSPR = L::QSPR, NSLOT = L::NSLOT;
  constexpr int OPS = 16 / NW;  // direct loads per wave and state piece
  static_assert(CWN == 2, "two column tiles per wave");
  constexpr int TS = L::TS, SPC = kChunk / TS, TT = TS / 16;  // rows per step, steps per chunk, token tiles
  static_assert(V % kWideCols == 0 && K == V && NSLOT >= 1 && NSLOT <= 4, "square heads of 128, 256 or 512");
  __shared__ __attribute__((aligned(1024))) char q_lds[2 * L::BYTES];
  // block b -> column tile (b / 8) % NH of unit (b % 8) + 8 (b / (8 NH)); a unit is (run, head)
  const int b = blockIdx.x;
  const int unit = (b & 7) + 8 * (b / (8 * NH));
  if (unit >= n_units) return;
  const int h = unit % H, tile = (b >> 3) % NH;
  // uniform values kept in scalar registers, so the chunk table reads are scalar loads
  const int c_begin = __builtin_amdgcn_readfirstlane((unit / H) * per);
  const int c_end = __builtin_amdgcn_readfirstlane(min(c_begin + per, n_chunk));
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int colw = tile * kWideCols + 16 * CWN * w;  // this wave's first column

  // step i (rows r0 .. r0 + TS - 1 of chunk c_begin + i / SPC, r0 = TS (i % SPC))
  // into buffer bi: the buffer is a flat run of 16-byte slots, row r's channels
  // 8 p .. 8 p + 7 in slot r QSPR + p; the spare slot of a row loads a copy of
  // its first piece, rows past the chunk end its last row
  auto stage = [&](int i, int bi) {
    const int c = c_begin + i / SPC, r0 = TS * (i % SPC);
    const int t0 = __builtin_amdgcn_readfirstlane(chunk_tok0[c]) + r0;
    const int ln = __builtin_amdgcn_readfirstlane(chunk_len[c]) - r0;
    if (ln <= 0) return;
    const __bf16* qh = q + (size_t)h * K;
    char* const dst = q_lds + bi * L::BYTES;
    // the lane index, opaque so that the per-load lane offsets are formed here
    // and not kept in registers across the step loop (spilled, their reloads
    // would wait for the direct loads in flight)
    int ql = lane;
    asm volatile("" : "+v"(ql));
#pragma unroll
    for (int u = 0; u < (L::NF + NW - 1) / NW; ++u) {
      const int f = NW * u + w;  // wave w: loads w, w + NW, ...
      if (f < L::NF) {
        const int sg = 64 * f + ql, row = min(min(sg / QSPR, TS - 1), ln - 1), piece = sg % QSPR;
        lds_dma16(qh + (size_t)(t0 + row) * H * K + 8 * (piece < K / 8 ? piece : 0), dst + f * 1024);
      }
    }
  };
  // A operand of step s, tile n: element j is
  // bf16(S)[32 s + 8 lg + j][colw + 8 (lr / 4) + 4 n + lr % 4] (row 4 g + e of tile n
  // is column 8 g + 4 n + e of the wave's 32, so that a lane ends with 8 adjacent
  // columns of one token)
  bf16x8 sr[KS][CWN];
  // The state reaches the registers through the free q buffer: rows
  // 32 p .. 32 p + 31 of the workgroup's 128 columns (16 KiB of fp32; one direct
  // load of 1 KiB covers two rows, 2 per wave) go to slot p % NSLOT, and each lane
  // then reads its 8 values of channel step p from there, with up to NSLOT - 1
  // later pieces in flight.
  auto load_sr = [&](int blk, char* free_buf) {
    const float* sp = snaps + ((size_t)(block_slot ? block_slot[blk] : blk) * H + h) * K * V +
                      (size_t)(lane >> 5) * V + tile * kWideCols + 4 * (lane & 31);
    auto stage_piece = [&](int pc) {
#pragma unroll
      for (int i = 0; i < OPS; ++i) {
        const int r2 = NW * i + w;  // rows 2 r2, 2 r2 + 1 of the piece
        lds_dma16(sp + (size_t)(32 * pc + 2 * r2) * V, free_buf + (pc % NSLOT) * L::PIECE + r2 * 1024);
      }
    };
    // this lane's word of a piece for tile n: row 8 lg + j, column colw - col0 + its column in the tile
    const int lcol = 8 * (lr >> 2) + (lr & 3);
    const __attribute__((address_space(3))) char* const rb =
        (const __attribute__((address_space(3))) char*)free_buf + (8 * lg * kWideCols + 16 * CWN * w + lcol) * 4;
#pragma unroll
    for (int pc = 0; pc < NSLOT - 1 && pc < KS; ++pc) stage_piece(pc);
#pragma unroll
    for (int pc = 0; pc < KS; ++pc) {
      if (pc + NSLOT - 1 < KS) stage_piece(pc + NSLOT - 1);
      // piece pc landed; the (2 per wave) loads of the pieces after it may still be in flight
      const int ahead = (KS - 1 - pc < NSLOT - 1) ? KS - 1 - pc : NSLOT - 1;
      if (ahead >= 3) vm_wait_barrier<3 * OPS>();
      else if (ahead == 2) vm_wait_barrier<2 * OPS>();
      else if (ahead == 1) vm_wait_barrier<OPS>();
      else vm_wait_barrier<0>();
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int n = 0; n < CWN; ++n)
          sr[pc][n][j] = (__bf16)*(const __attribute__((address_space(3))) float*)(
              rb + (pc % NSLOT) * L::PIECE + j * kWideCols * 4 + 16 * n);
      // every wave's reads of the slot done before a later piece lands there
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
  };

  const int n_steps = (c_end - c_begin) * SPC;
  stage(0, 0);
  vm_wait_barrier<0>();  // the first step's rows are in LDS
  int sr_block = -1;
  for (int i = 0; i < n_steps; ++i) {
    const int bi = i & 1, c = c_begin + i / SPC, r0 = TS * (i % SPC);
    const int tok0 = __builtin_amdgcn_readfirstlane(chunk_tok0[c]) + r0;
    const int len = __builtin_amdgcn_readfirstlane(chunk_len[c]) - r0;  // rows of this step: min(len, TS)
    const int blk = __builtin_amdgcn_readfirstlane(block_ids[c]);
    // a new block's state, through the other buffer (free: its reads ended
    // before the last barrier) before the next chunk's rows go there
    if (len > 0 && blk != sr_block) {
      load_sr(blk, q_lds + (bi ^ 1) * L::BYTES);
      sr_block = blk;
    }
    // the next step's rows into the other buffer
    if (i + 1 < n_steps) stage(i + 1, bi ^ 1);
    f32x4 acc[TT][CWN];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int n = 0; n < CWN; ++n) acc[tt][n] = zero4();
    if (len > 0) {
      // this lane's q operand: token 16 tt + lr, channels 32 s + 8 lg .. + 7 (its
      // offset formed here from an opaque lane index: a value kept across the
      // step loop would be spilled, and its reload would wait for the next
      // step's direct loads)
      int ml = lane;
      asm volatile("" : "+v"(ml));
      const __attribute__((address_space(3))) char* const qb =
          (const __attribute__((address_space(3))) char*)q_lds + bi * L::BYTES + ((ml & 15) * QSPR + (ml >> 4)) * 16;
      // the operands in batches of 8 reads, all issued before the batch's products
      // (left to itself the compiler waited for each read before its two products;
      // 0.36 -> 0.34 ms at d = 512, 64 heads and 8192 tokens)
      constexpr int SB = 8 / TT;  // channel steps per batch
      static_assert(KS % SB == 0, "channel steps in whole batches");
#pragma unroll
      for (int s0 = 0; s0 < KS; s0 += SB) {
        bf16x8 qv[SB][TT];
#pragma unroll
        for (int ds = 0; ds < SB; ++ds)
#pragma unroll
          for (int tt = 0; tt < TT; ++tt)
            qv[ds][tt] = *(const __attribute__((address_space(3))) bf16x8*)(qb + (16 * tt * QSPR + 4 * (s0 + ds)) * 16);
        __builtin_amdgcn_sched_barrier(0);  // keep the batch's reads together
#pragma unroll
        for (int ds = 0; ds < SB; ++ds)
#pragma unroll
          for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int n = 0; n < CWN; ++n) acc[tt][n] = mfma_bf16(sr[s0 + ds][n], qv[ds][tt], acc[tt][n]);
      }
    }
    // every wave's loads of the next step landed, every wave done with this buffer
    // (the wait also covers the previous step's stores, long since issued)
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (len > 0) {
      int sl = lane;  // opaque again: the row offsets are formed here
      asm volatile("" : "+v"(sl));
      __bf16* const op = o + ((size_t)tok0 * H + h) * V + colw + 4 * CWN * (sl >> 4);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const int t = 16 * tt + (sl & 15);
        if (t < len) {
          bf16x8 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = (__bf16)(acc[tt][0][e] * scale);
            v[4 + e] = (__bf16)(acc[tt][1][e] * scale);
          }
          *(bf16x8*)(op + (size_t)t * H * V) = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The epilogue of MemTRMSNormGated (models/qwen/layer.py:22-31) applied to one
// value of a row whose mean square is `ms`:
//   y = bf16(x * rsqrt(ms + eps)); y = bf16(w * y); out = bf16(y * gate_fn(g)).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float gate_value(float g, float softcap, int gate_kind) {
  if (gate_kind == MEMT_GDN2_GATE_SIGMOID) return 1.f / (1.f + expf(-g));
  const float silu = g / (1.f + expf(-g));
  return softcap * tanhf(silu / softcap);
}

__device__ __forceinline__ __bf16 norm_gate_one(float x, float rs, float wt, float g, float softcap,
                                                int gate_kind) {
  const float y = (float)(__bf16)(x * rs);
  const float yw = (float)(__bf16)(wt * y);
  return (__bf16)(yw * gate_value(g, softcap, gate_kind));
}

// ---------------------------------------------------------------------------
// Fused decode readout: one workgroup per (sequence, head).
//   r = bf16(scale * q . S) (fp32 S, fp32 accumulation), then the epilogue.
// Options (ReadoutArgs::flags):
//   MEMT_GDN2_READOUT_L2NORM_Q  q is the raw projection row: the kernel forms
//                               q_hat = bf16(q / sqrt(sum q^2 + q_eps)) first
//                               (FLA l2norm_fwd, as the block's query path does);
//   STATE_BF16 (template)       the dot reads bf16(S), the reference reader's
//                               operand rounding (models/qwen/ops/_triton/read.py:64).
// Thread (rg, cg) streams rows rg, rg + RG, rg + 2RG, ... of columns
// [4cg, 4cg+4) with 16-byte loads, so one wave instruction reads 64 / CG
// whole adjacent rows.  Every global load (q, gate, weight and the first NB
// state rows) is issued before the first wait, and the waits are LDS-only
// barriers, so the state stream starts at once; with more than NB rows per
// thread each consumed row is replaced by the next one (a rolling window).
// ---------------------------------------------------------------------------
// Threads of a readout workgroup: one per value column at d = 512.
__host__ __device__ constexpr int readout_threads(int V) { return V > 256 ? V : 256; }

template <int K, int V, bool STATE_BF16>
__global__ __launch_bounds__(readout_threads(V)) void readout_kernel(ReadoutArgs a) {
  constexpr int NT = readout_threads(V);
  constexpr int CG = V / 4;          // float4 column groups
  constexpr int RG = NT / CG;        // row groups
  constexpr int RPT = K / RG;        // rows per thread
  constexpr int NB = RPT < 16 ? RPT : 16;  // state rows in flight per thread
  static_assert(RG * CG == NT && RPT * RG == K && RPT % NB == 0 && K <= NT, "readout tiling");
  __shared__ float q_s[NT];  // every thread stores: no branch before the first wait
  __shared__ float part[RG][V];
  __shared__ float red[NT / 64];
  __shared__ float qred[NT / 64];
  const int H = a.H;
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int tid = threadIdx.x;
  const int slot = a.slot_idx ? a.slot_idx[b] : b;
  const float* Sp = a.S + ((size_t)slot * H + h) * K * V;
  const int cg = tid % CG, rg = tid / CG;
  // clamped indices keep these loads unconditional
  const float qv = (float)a.q[(size_t)b * a.q_stride + (size_t)h * K + (tid < K ? tid : K - 1)];
  const float gv = (float)a.gate[(size_t)b * a.gate_stride + (size_t)h * V + (tid < V ? tid : V - 1)];
  const float wv = (float)a.weight[tid < V ? tid : V - 1];
  asm volatile("" ::: "memory");  // issue q before the state rows: its wait then leaves them in flight
  f32x4 s4[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
    s4[i] = __builtin_nontemporal_load((const f32x4*)(Sp + (size_t)(i * RG + rg) * V + 4 * cg));
  float qn = qv;
  if (a.flags & MEMT_GDN2_READOUT_L2NORM_Q) {
    // the query's l2 norm over its K channels (threads past K hold a clamped copy: excluded)
    const float qsq = wave_sum(tid < K ? qv * qv : 0.f);
    if ((tid & 63) == 0) qred[tid >> 6] = qsq;
    lds_barrier();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < (K + 63) / 64; ++i) tot += qred[i];
    qn = (float)(__bf16)(qv * (1.f / sqrtf(tot + a.q_eps)));
  }
  q_s[tid] = qn;
  lds_barrier();
  f32x4 acc = zero4();
#pragma unroll
  for (int j = 0; j < RPT / NB; ++j) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int k = (j * NB + i) * RG + rg;
      const float qk = q_s[k];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(qk, STATE_BF16 ? (float)(__bf16)s4[i][e] : s4[i][e], acc[e]);
      if (j + 1 < RPT / NB)
        s4[i] = __builtin_nontemporal_load((const f32x4*)(Sp + (size_t)(k + NB * RG) * V + 4 * cg));
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) part[rg][4 * cg + e] = acc[e];
  lds_barrier();
  float r = 0.f, sq = 0.f;
  if (tid < V) {
    float sum = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < RG; ++g2) sum += part[g2][tid];
    r = (float)(__bf16)(sum * a.scale);  // the reader's bf16 output
    sq = r * r;
  }
  sq = wave_sum(sq);
  if ((tid & 63) == 0) red[tid >> 6] = sq;
  lds_barrier();
  if (tid < V) {
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < (V + 63) / 64; ++i) tot += red[i];
    const float rs = rsqrtf(tot / (float)V + a.eps);
    a.out[((size_t)b * H + h) * V + tid] = norm_gate_one(r, rs, wv, gv, a.softcap, a.gate_kind);
  }
}

// MemTRMSNormGated over rows of `dim` (one wave per row, dim <= 1024).
__global__ __launch_bounds__(256) void rms_norm_gated_kernel(const __bf16* __restrict__ x,
                                                             const __bf16* __restrict__ gate,
                                                             const __bf16* __restrict__ weight,
                                                             __bf16* __restrict__ out, int64_t rows,
                                                             int dim, float eps, float softcap,
                                                             int gate_kind) {
  const int64_t rrow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (rrow >= rows) return;
  const __bf16* xr = x + rrow * dim;
  float vals[16];
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = lane + 64 * i;
    vals[i] = (c < dim) ? (float)xr[c] : 0.f;
    sq += vals[i] * vals[i];
  }
  sq = wave_sum(sq);
  const float rs = rsqrtf(sq / (float)dim + eps);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = lane + 64 * i;
    if (c < dim)
      out[rrow * dim + c] =
          norm_gate_one(vals[i], rs, (float)weight[c], (float)gate[rrow * dim + c], softcap, gate_kind);
  }
}

// FLA l2norm_fwd (FLA/modules/l2norm.py:95-109): one wave per row, dim <= 512.
template <bool XBF, bool YBF>
__global__ __launch_bounds__(256) void l2norm_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                     float* __restrict__ rstd, int64_t rows, int dim,
                                                     float eps) {
  const int64_t rrow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (rrow >= rows) return;
  float vals[8];
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = lane + 64 * i;
    float v = 0.f;
    if (c < dim) v = XBF ? (float)((const __bf16*)x)[rrow * dim + c] : ((const float*)x)[rrow * dim + c];
    vals[i] = v;
    sq += v * v;
  }
  sq = wave_sum(sq);
  const float rs = 1.f / sqrtf(sq + eps);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = lane + 64 * i;
    if (c < dim) {
      const float v = vals[i] * rs;
      if (YBF)
        ((__bf16*)y)[rrow * dim + c] = (__bf16)v;
      else
        ((float*)y)[rrow * dim + c] = v;
    }
  }
  if (rstd != nullptr && lane == 0) rstd[rrow] = rs;
}

// Chunk-local cumsum (FLA/ops/utils/cumsum.py:116-133): one thread per
// (chunk, head, channel), sequential over the chunk's tokens.
template <bool GBF>
__global__ __launch_bounds__(256) void cumsum_kernel(const void* __restrict__ g, float* __restrict__ gk,
                                                     const int32_t* chunk_tok0, const int32_t* chunk_len,
                                                     int H, int S, float scale, int reverse) {
  const int chunk = blockIdx.x, h = blockIdx.y;
  const int c = blockIdx.z * 256 + threadIdx.x;
  if (c >= S) return;
  const int tok0 = chunk_tok0[chunk], len = chunk_len[chunk];
  float run = 0.f;
  for (int i = 0; i < len; ++i) {
    const int t = reverse ? (len - 1 - i) : i;
    const size_t off = ((size_t)(tok0 + t) * H + h) * S + c;
    run += GBF ? (float)((const __bf16*)g)[off] : ((const float*)g)[off];
    gk[off] = run * scale;
  }
}

// Workspace fragments -> the reference's [T, H, D] bf16 layouts.
template <int K, int V>
__global__ __launch_bounds__(256) void wy_export_kernel(WyBuffers in, const int32_t* chunk_tok0,
                                                        const int32_t* chunk_len, int H, __bf16* w,
                                                        __bf16* u, __bf16* kg, __bf16* Aqk, __bf16* qg) {
  constexpr int C = kChunk;
  const int chunk = blockIdx.x, h = blockIdx.y;
  const size_t unit = (size_t)chunk * H + h;
  const int tok0 = chunk_tok0[chunk], len = chunk_len[chunk];
  for (int idx = threadIdx.x; idx < len * K; idx += 256) {
    const int t = idx / K, c = idx % K;
    const size_t dst = ((size_t)(tok0 + t) * H + h) * K + c;
    if (w) w[dst] = (__bf16)(float)in.W[unit * C * K + pfrag_index(t, c, K)];
    if (kg) kg[dst] = (__bf16)(float)in.kgT[unit * C * K + pfrag_index(c, t, C)];
    if (qg && in.qg) qg[dst] = (__bf16)(float)in.qg[unit * C * K + pfrag_index(t, c, K)];
  }
  constexpr int NP = wy_passes(K);
  for (int idx = threadIdx.x; idx < len * V; idx += 256) {
    const int t = idx / V, c = idx % V;
    const float us = ldexpf(1.f, in.uexp[unit * NP + c / (V / NP)]);  // U is stored as U * 2^-uexp
    if (u) u[((size_t)(tok0 + t) * H + h) * V + c] = (__bf16)((float)in.U[unit * C * V + cfrag_index(t, c, V)] * us);
  }
  if (Aqk && in.Aqk) {
    for (int idx = threadIdx.x; idx < len * C; idx += 256) {
      const int t = idx / C, j = idx % C;
      Aqk[((size_t)(tok0 + t) * H + h) * C + j] = (__bf16)(float)in.Aqk[unit * C * C + pfrag_index(t, j, C)];
    }
  }
}

// The reference's [T, H, D] WY tensors -> workspace fragments (rows past the
// chunk end are zero), decay = 2^{gk at the chunk's last token}.
template <int K, int V>
__global__ __launch_bounds__(256) void wy_import_kernel(const __bf16* w, const __bf16* u, const __bf16* kg,
                                                        const float* gk, const int32_t* chunk_tok0,
                                                        const int32_t* chunk_len, int H, WyBuffers out) {
  constexpr int C = kChunk;
  const int chunk = blockIdx.x, h = blockIdx.y;
  const size_t unit = (size_t)chunk * H + h;
  const int tok0 = chunk_tok0[chunk], len = chunk_len[chunk];
  for (int idx = threadIdx.x; idx < C * K; idx += 256) {
    const int t = idx / K, c = idx % K;
    const size_t src = ((size_t)(tok0 + t) * H + h) * K + c;
    const bool ok = t < len;
    out.W[unit * C * K + pfrag_index(t, c, K)] = (_Float16)(ok ? (float)w[src] : 0.f);
    out.kgT[unit * C * K + pfrag_index(c, t, C)] = (_Float16)(ok ? (float)kg[src] : 0.f);
  }
  // U goes to f16 as U * 2^-uexp, uexp the value exponent of each channel pass's max |U|
  constexpr int NP = wy_passes(K), VP = V / NP;
  __shared__ float red[4];
  for (int p = 0; p < NP; ++p) {
    float m = 0.f;
    for (int idx = threadIdx.x; idx < len * VP; idx += 256) {
      const int t = idx / VP, c = p * VP + idx % VP;
      m = fmaxf(m, fabsf((float)u[((size_t)(tok0 + t) * H + h) * V + c]));
    }
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    const int uexp = value_exponent(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
    __syncthreads();  // red is reused by the next pass
    const float us = ldexpf(1.f, -uexp);
    if (threadIdx.x == 0) out.uexp[unit * NP + p] = uexp;
    for (int idx = threadIdx.x; idx < C * VP; idx += 256) {
      const int t = idx / VP, c = p * VP + idx % VP;
      const bool ok = t < len;
      out.U[unit * C * V + cfrag_index(t, c, V)] =
          (_Float16)(ok ? (float)u[((size_t)(tok0 + t) * H + h) * V + c] * us : 0.f);
    }
  }
  for (int c = threadIdx.x; c < K; c += 256)
    out.decay[unit * K + c] = fast_exp2(gk[((size_t)(tok0 + len - 1) * H + h) * K + c]);
}

}  // namespace

// CUs of the current device, looked up once per device (callers on several host
// threads may race to fill an entry; they store the same value)
static int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

hipError_t launch_read_fwd(const __bf16* q, const float* snaps, __bf16* o, const int32_t* chunk_tok0,
                           const int32_t* chunk_len, const int32_t* chunk_block_ids, int n_chunk, int H,
                           int K, int V, float scale, hipStream_t stream, const int32_t* block_slot) {
  if (n_chunk == 0) return hipSuccess;
#define MEMT_RD(KK, VV)                                                                                        \
  if (K == KK && V == VV) {                                                                                    \
    const int n_units = (n_chunk + kReadRun - 1) / kReadRun * H;                                               \
    hipLaunchKernelGGL((read_fwd_kernel<KK, VV>), dim3(n_units), dim3(256), 0, stream, q, snaps, o, chunk_tok0,  \
                       chunk_len, chunk_block_ids, n_chunk, n_units, H, scale, block_slot);                    \
    return hipGetLastError();                                                                                  \
  }
  MEMT_RD(64, 64)
#undef MEMT_RD
  if (K == V && (K == 128 || K == 256 || K == 512)) {
    // runs sized so the grid fills the chip once
    const int nh = V / kWideCols, per_run = H * nh, slots = device_cus() * wide_per_cu(K);
    const int runs_wanted = (slots + per_run - 1) / per_run;  // at least 1
    // (at d = 128 a run's state, 64 KB, is two chunks' q and o: runs of at least
    // kReadRun chunks keep the state reloads to a third of the traffic)
    const int per = std::max((n_chunk + runs_wanted - 1) / runs_wanted, K == 128 ? kReadRun : 1);
    const int n_units = (n_chunk + per - 1) / per * H;
    const int n_blocks = (n_units + 7) / 8 * 8 * nh;
    if (K == 128)
      hipLaunchKernelGGL((read_wide_kernel<128, 128>), dim3(n_blocks), dim3(64 * kWideWaves), 0, stream, q, snaps, o,
                         chunk_tok0, chunk_len, chunk_block_ids, n_chunk, n_units, per, H, scale, block_slot);
    else if (K == 256)
      hipLaunchKernelGGL((read_wide_kernel<256, 256>), dim3(n_blocks), dim3(64 * kWideWaves), 0, stream, q, snaps, o,
                         chunk_tok0, chunk_len, chunk_block_ids, n_chunk, n_units, per, H, scale, block_slot);
    else
      hipLaunchKernelGGL((read_wide_kernel<512, 512>), dim3(n_blocks), dim3(64 * kWideWaves), 0, stream, q, snaps, o,
                         chunk_tok0, chunk_len, chunk_block_ids, n_chunk, n_units, per, H, scale, block_slot);
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

hipError_t launch_readout(const ReadoutArgs& a, int B, int K, int V, bool state_bf16, hipStream_t stream) {
  if (B == 0) return hipSuccess;
  dim3 grid(B * a.H);
#define MEMT_RO(KK, VV)                                                                                      \
  if (K == KK && V == VV) {                                                                                  \
    if (state_bf16)                                                                                          \
      hipLaunchKernelGGL((readout_kernel<KK, VV, true>), grid, dim3(readout_threads(VV)), 0, stream, a);     \
    else                                                                                                     \
      hipLaunchKernelGGL((readout_kernel<KK, VV, false>), grid, dim3(readout_threads(VV)), 0, stream, a);    \
    return hipGetLastError();                                                                                \
  }
  MEMT_RO(64, 64)
  MEMT_RO(128, 128)
  MEMT_RO(256, 256)
  MEMT_RO(512, 512)
#undef MEMT_RO
  return hipErrorInvalidValue;
}

hipError_t launch_rms_norm_gated(const __bf16* x, const __bf16* gate, const __bf16* weight, __bf16* out,
                                 int64_t rows, int dim, float eps, float softcap, int gate_kind,
                                 hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  hipLaunchKernelGGL(rms_norm_gated_kernel, grid, block, 0, stream, x, gate, weight, out, rows, dim, eps, softcap,
                     gate_kind);
  return hipGetLastError();
}

hipError_t launch_l2norm(const void* x, bool x_bf16, void* y, bool y_bf16, float* rstd, int64_t rows, int dim,
                         float eps, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  if (x_bf16 && y_bf16)
    hipLaunchKernelGGL((l2norm_kernel<true, true>), grid, block, 0, stream, x, y, rstd, rows, dim, eps);
  else if (x_bf16 && !y_bf16)
    hipLaunchKernelGGL((l2norm_kernel<true, false>), grid, block, 0, stream, x, y, rstd, rows, dim, eps);
  else if (!x_bf16 && y_bf16)
    hipLaunchKernelGGL((l2norm_kernel<false, true>), grid, block, 0, stream, x, y, rstd, rows, dim, eps);
  else
    hipLaunchKernelGGL((l2norm_kernel<false, false>), grid, block, 0, stream, x, y, rstd, rows, dim, eps);
  return hipGetLastError();
}

hipError_t launch_cumsum(const void* g, bool g_bf16, float* gk, const int32_t* chunk_tok0,
                         const int32_t* chunk_len, int n_chunk, int H, int S, float scale, bool reverse,
                         hipStream_t stream) {
  if (n_chunk == 0) return hipSuccess;
  dim3 grid(n_chunk, H, (S + 255) / 256), block(256);
  if (g_bf16)
    hipLaunchKernelGGL((cumsum_kernel<true>), grid, block, 0, stream, g, gk, chunk_tok0, chunk_len, H, S, scale,
                       reverse ? 1 : 0);
  else
    hipLaunchKernelGGL((cumsum_kernel<false>), grid, block, 0, stream, g, gk, chunk_tok0, chunk_len, H, S, scale,
                       reverse ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_wy_export(const WyBuffers& in, const int32_t* chunk_tok0, const int32_t* chunk_len, int n_chunk,
                            int H, int K, int V, __bf16* w, __bf16* u, __bf16* kg, __bf16* Aqk, __bf16* qg,
                            hipStream_t stream) {
  if (n_chunk == 0) return hipSuccess;
  dim3 grid(n_chunk, H), block(256);
  if (K == 64 && V == 64)
    hipLaunchKernelGGL((wy_export_kernel<64, 64>), grid, block, 0, stream, in, chunk_tok0, chunk_len, H, w, u, kg,
                       Aqk, qg);
  else if (K == 128 && V == 128)
    hipLaunchKernelGGL((wy_export_kernel<128, 128>), grid, block, 0, stream, in, chunk_tok0, chunk_len, H, w, u, kg,
                       Aqk, qg);
  else if (K == 256 && V == 256)
    hipLaunchKernelGGL((wy_export_kernel<256, 256>), grid, block, 0, stream, in, chunk_tok0, chunk_len, H, w, u, kg,
                       Aqk, qg);
  else if (K == 512 && V == 512)
    hipLaunchKernelGGL((wy_export_kernel<512, 512>), grid, block, 0, stream, in, chunk_tok0, chunk_len, H, w, u, kg,
                       Aqk, qg);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_wy_import(const __bf16* w, const __bf16* u, const __bf16* kg, const float* gk,
                            const int32_t* chunk_tok0, const int32_t* chunk_len, int n_chunk, int H, int K, int V,
                            WyBuffers out, hipStream_t stream) {
  if (n_chunk == 0) return hipSuccess;
  dim3 grid(n_chunk, H), block(256);
  if (K == 64 && V == 64)
    hipLaunchKernelGGL((wy_import_kernel<64, 64>), grid, block, 0, stream, w, u, kg, gk, chunk_tok0, chunk_len, H,
                       out);
  else if (K == 128 && V == 128)
    hipLaunchKernelGGL((wy_import_kernel<128, 128>), grid, block, 0, stream, w, u, kg, gk, chunk_tok0, chunk_len, H,
                       out);
  else if (K == 256 && V == 256)
    hipLaunchKernelGGL((wy_import_kernel<256, 256>), grid, block, 0, stream, w, u, kg, gk, chunk_tok0, chunk_len, H,
                       out);
  else if (K == 512 && V == 512)
    hipLaunchKernelGGL((wy_import_kernel<512, 512>), grid, block, 0, stream, w, u, kg, gk, chunk_tok0, chunk_len, H,
                       out);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace memt
