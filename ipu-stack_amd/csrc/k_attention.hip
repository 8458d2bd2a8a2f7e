// Fused online-softmax attention on gfx950 MFMA:
//   O = softmax(scale * Q K^T [+ causal mask]) V
// Q, K, V fp16 [streams, rows, width]; fp32 scores, running max and sum;
// fp32 output by default (the reference's device attention output precision,
// crates/ipu-codegen/src/mid.rs:2064-2067) or fp16.  Semantics:
// device/flash_attention_online_f16.cpp:68-143 (online softmax, exact) and
// crates/ipu-tests/src/diagnostic.rs:711-780 (key j allowed iff j <= i when
// causal, 741-745; scale default 1/sqrt(width), 733-736).
//
// Fast kernel (width == value width, a multiple of 8 up to 128, computed in
// tiles 64 or 128 columns wide with zero padding):
//   * 256 threads = 4 waves; a wave owns 32 queries, a workgroup 128 queries
//     of one stream; two workgroups share a CU (launch bound), so one SIMD
//     runs the softmax of one wave while the MFMA pipe serves the other;
//   * keys stream through LDS in blocks of 64 with two stages.  K and V tiles
//     are copied global -> LDS with buffer_load ... lds (16 bytes per lane, no
//     staging registers; rows past the end of the stream read as 0), both
//     stored row-major [64 keys][D] with an XOR swizzle of 16-byte chunks;
//   * software pipeline: step j runs ONE MFMA cluster holding the scores of
//     block j and the output update of block j - 1 (alternating, fragments
//     read ahead, the step's DMA instructions spread between them), then the
//     softmax of block j on the VALU.  K tiles run one block ahead of V;
//   * scores are computed transposed, S^T = K Q^T, with
//     v_mfma_f32_32x32x16_f16 (K fragments by ds_read_b128 as the first
//     operand, Q fragments resident in registers as the second), so a lane
//     holds 32 keys of ONE query: the row max needs one exchange (lane ^ 32)
//     and the running sum none until the end;
//   * the output is accumulated transposed, O^T += V^T P^T: the fp16
//     probabilities are the second MFMA operand straight from the score
//     registers, and the matching V^T fragments come from the row-major V
//     tile through ds_read_b64_tr_b16, whose 4-key runs are chosen to follow
//     the score accumulator's key order;
//   * the reference point (running max) moves only when some probability of
//     a block would exceed 2^kRescaleSlack, which the block's probability
//     sum bounds, so no max over the scores is taken on the common path:
//     the result is exact for any reference point, and most blocks skip the
//     max, the rescale of the output accumulators and the exchange with the
//     partner lane;
//   * K and V fragment offsets are computed once per lane (XOR swizzles of
//     one base), so the cluster's LDS reads take immediate offsets only;
//   * causal: key blocks past the workgroup's last query are never loaded, a
//     wave skips blocks past its own last query.
//   * causal: one workgroup runs query blocks n - 1 - i and then i of one
//     stream, so every workgroup has the same number of key steps;
//     workgroups are remapped so each XCD (round-robin dispatch over 8) runs
//     whole streams, sharing K and V in its L2.
#include "../../include/ipus.h"
#include "device_common.h"
#include "kernels.h"

#define LDS_AS __attribute__((address_space(3)))

namespace ipus {
namespace {

constexpr int kThreads = 256;
constexpr int kQueriesPerWave = 32;
constexpr int kQueriesPerBlock = 128;
constexpr int kKeysPerBlock = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.0f;
constexpr float kSumLimit = 256.0f;  // 2^kRescaleSlack
constexpr int kBufferFlags = 0x00020000;  // raw buffer, dword 3 of the descriptor

typedef short short4_t __attribute__((vector_size(8)));

inline int hip_status(hipError_t e) { return e == hipSuccess ? 0 : IPUS_ERROR_HIP_BASE - (int)e; }

// Tiles of 64 keys x D fp16, rows of D * 2 bytes, 16-byte chunks swizzled by
// row.  K is read with ds_read_b128 (16 consecutive rows, one chunk, per
// 256-byte cycle); V with ds_read_b64_tr_b16 (4 consecutive rows x 4 chunks
// per 32 lanes).  The XORs give each of those reads distinct banks.
template <int D>
struct KvTile {
  static constexpr uint32_t kRowBytes = D * 2;
  static constexpr uint32_t kChunks = D / 8;
  static constexpr uint32_t kBytes = kKeysPerBlock * D * 2;
  static constexpr uint32_t kDma = kBytes / 16 / kThreads;  // DMA instructions per thread
};
template <int D>
__device__ __forceinline__ uint32_t k_swz(uint32_t row) {
  return D == 128 ? (row & 15u) : ((row >> 1) & 7u);
}
template <int D>
__device__ __forceinline__ uint32_t v_swz(uint32_t row) {
  return D == 128 ? ((row & 3u) << 2) : (((row >> 1) & 1u) << 2);
}
template <int D>
__device__ __forceinline__ uint32_t k_off(uint32_t row, uint32_t chunk) {
  return row * KvTile<D>::kRowBytes + ((chunk ^ k_swz<D>(row)) << 4);
}
template <int D>
__device__ __forceinline__ uint32_t v_off(uint32_t row, uint32_t chunk) {
  return row * KvTile<D>::kRowBytes + ((chunk ^ v_swz<D>(row)) << 4);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// max / sum of x over lanes l and l ^ 32 (one ds_bpermute exchange).
__device__ __forceinline__ float max_with_partner(float x) {
  return fmaxf(x, __shfl_xor(x, 32, kWave));
}
__device__ __forceinline__ float sum_with_partner(float x) { return x + __shfl_xor(x, 32, kWave); }

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LDS_AS void*)lds, 16, voffset, 0, 0, 0);
}

// Byte offset within a key block of the chunk this thread's first DMA
// instruction fetches: instruction i of thread t fills LDS slot i * 256 + t,
// so it loads the chunk that the swizzle places there.  Instruction i covers
// the rows kThreads / kChunks * i further on with the same swizzled chunk (the
// swizzles depend only on row bits that this step leaves alone), so the other
// instructions add a wave-uniform row offset.  row_bytes is the global row
// pitch: width * 2 for a contiguous [streams, rows, width] tensor, heads *
// width * 2 for a head of an unsplit [batch, rows, heads * width].  Chunks at
// or past the width (a width below the tile's D, padded) get an offset past
// the buffer's range, so their loads return 0: kPadOffset plus any block
// offset (< 2^31) stays above the range (< 0x7fff0000) without wrapping.
constexpr uint32_t kPadOffset = 0x80000000u;
template <int D, bool IsK>
__device__ __forceinline__ uint32_t kv_offset(uint32_t row_bytes, uint32_t width) {
  const uint32_t row = threadIdx.x / KvTile<D>::kChunks, phys = threadIdx.x % KvTile<D>::kChunks;
  const uint32_t chunk = phys ^ (IsK ? k_swz<D>(row) : v_swz<D>(row));
  return chunk * 8 < width ? row * row_bytes + chunk * 16 : kPadOffset;
}

template <int D, bool Causal, bool OutF16>
__device__ __forceinline__ void attention_block(
    void* __restrict__ out, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, uint32_t stream, uint32_t qb, uint32_t query_rows,
    uint32_t key_rows, uint32_t width, float scale_log2, uint32_t q_heads, uint32_t k_heads,
    uint32_t v_heads) {
  constexpr uint32_t kDT = D / 32;  // output d tiles
  constexpr uint32_t kKS = D / 16;  // k steps of the score MFMA
  constexpr uint32_t kTile = KvTile<D>::kBytes;
  constexpr uint32_t kDmaRows = kThreads / KvTile<D>::kChunks;  // rows per DMA instruction
  static_assert(4 * kDT == 2 * kKS, "one PV MFMA per score MFMA");
  // Two stages, each a distinct LDS object so the compiler can see that the
  // DMA into one stage never aliases the fragment reads of the other.
  __shared__ __attribute__((aligned(1024))) uint8_t lds_k0[kTile];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_v0[kTile];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_k1[kTile];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_v1[kTile];

  const uint32_t q0 = qb * kQueriesPerBlock;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave_s = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const uint32_t wq0 = q0 + wave_s * kQueriesPerWave;  // first query of this wave

  // Stream s of an operand with h heads is head s % h of matrix s / h of a
  // [streams / h, rows, h * D] tensor (h = 1: contiguous [streams, rows, D]).
  // The tile width D is the stream width padded to 64 or 128.
  const uint32_t q_pitch = q_heads * width;
  const uint32_t k_row_bytes = k_heads * width * 2u, v_row_bytes = v_heads * width * 2u;
  const uint16_t* Q = query + (uint64_t)(stream / q_heads) * query_rows * q_pitch + (stream % q_heads) * width;
  const uint16_t* K = key + (uint64_t)(stream / k_heads) * key_rows * k_heads * width + (stream % k_heads) * width;
  const uint16_t* V = value + (uint64_t)(stream / v_heads) * key_rows * v_heads * width + (stream % v_heads) * width;
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)K, 0, (int)((key_rows - 1) * k_row_bytes + width * 2u), kBufferFlags);
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)V, 0, (int)((key_rows - 1) * v_row_bytes + width * 2u), kBufferFlags);
  const uint32_t k_voff = kv_offset<D, true>(k_row_bytes, width);
  const uint32_t v_voff = kv_offset<D, false>(v_row_bytes, width);

  uint32_t key_end = key_rows;
  if (Causal) {
    const uint32_t last_q = q0 + kQueriesPerBlock < query_rows ? q0 + kQueriesPerBlock : query_rows;
    key_end = last_q < key_rows ? last_q : key_rows;  // keys <= last query
  }
  const uint32_t nblocks = (key_end + kKeysPerBlock - 1) / kKeysPerBlock;
  const uint32_t k_block_bytes = kKeysPerBlock * k_row_bytes;
  const uint32_t v_block_bytes = kKeysPerBlock * v_row_bytes;
  // Blocks this wave computes scores for (causal: keys <= its last query).
  // Every such block holds at least one allowed key per query of the wave.
  uint32_t nproc = nblocks;
  if (Causal) {
    const uint32_t lim = (wq0 + kQueriesPerWave - 1) / kKeysPerBlock + 1;
    nproc = lim < nproc ? lim : nproc;
  }

  // Q fragments (second MFMA operand): lane holds Q[q][16 ks + 8 (lane/32) ..+7].
  half8_t qf[kKS];
  {
    uint32_t q = wq0 + lane % 32;
    q = q < query_rows ? q : query_rows - 1;
#pragma unroll
    for (uint32_t ks = 0; ks < kKS; ++ks)
    {
      const uint32_t d0 = ks * 16 + (lane / 32) * 8;  // padding columns are 0
      qf[ks] = __builtin_bit_cast(
          half8_t, d0 < width ? load16(Q + (uint64_t)q * q_pitch + d0) : u32x4{0, 0, 0, 0});
    }
  }

  float16_t o[kDT];
#pragma unroll
  for (uint32_t dt = 0; dt < kDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m_run = -INFINITY;  // reference point, log2 units (scaled)
  float l_run = 0.0f;       // this lane's share of the row sum
  half8_t pp[2][2];         // fp16 probabilities of the last softmax
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) pp[st][h][e] = (half_t)0.0f;  // "block -1"
  const uint32_t qi = wq0 + lane % 32;

  // Fragment reads.  K fragment (first operand of S^T = K Q^T): lane holds
  // K[32 st + lane % 32][16 ks + 8 (lane / 32) .. +7].  V^T fragment (first
  // operand of O^T += V^T P^T) for d tile dt and keys 32 st + 16 h + {0..15}:
  // lane holds d = 32 dt + lane % 32 and, in element e, key 32 st + 16 h +
  // 8 (e / 4) + 4 (lane / 32) + e % 4, the key order of score accumulator
  // elements 8 h .. 8 h + 7; each ds_read_b64_tr_b16 returns 4 consecutive
  // keys (in a 16-lane group, source lane s addresses row key0 + s / 4,
  // columns d0 + 4 (s % 4) .. +3).  Offsets are those of the first rows
  // XORed with the k step (chunk 2 ks: bits 5..) or d tile (chunk 4 dt: bits
  // 6..), since both swizzles XOR the chunk with row bits; other rows add a
  // constant (an immediate offset of the LDS read).  The per-k-step and
  // per-d-tile offsets are computed once and stay in registers.
  const uint32_t kbase = k_off<D>(lane % 32, lane / 32);
  uint32_t vbase;
  {
    const uint32_t sl = lane % 16, g = lane / 32, dg = (lane / 16) % 2;
    const uint32_t d = 16 * dg + 4 * (sl % 4);
    vbase = v_off<D>(4 * g + sl / 4, d / 8) + (d % 8) * 2;
  }
  uint32_t kofs[kKS], vofs[kDT];
#pragma unroll
  for (uint32_t ks = 0; ks < kKS; ++ks) kofs[ks] = kbase ^ (ks << 5);
#pragma unroll
  for (uint32_t dt = 0; dt < kDT; ++dt) vofs[dt] = vbase ^ (dt << 6);
  auto kfrag = [&](const uint8_t* lk, uint32_t st, uint32_t ks) __attribute__((always_inline)) {
    const uint8_t* p = lk + kofs[ks] + st * 32 * KvTile<D>::kRowBytes;
    return __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4*>(p));
  };
  auto vfrag = [&](const uint8_t* lv, uint32_t st, uint32_t h, uint32_t dt) __attribute__((always_inline)) {
    const uint8_t* p = lv + vofs[dt] + (32 * st + 16 * h) * KvTile<D>::kRowBytes;
    const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)p);
    const short4_t hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)(p + 8 * KvTile<D>::kRowBytes));
    return __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  // DMA instruction i of a K or V tile.  The scalar part is opaque so the
  // per-instruction offsets are not hoisted out of the loop into registers;
  // the block offset stays in the vector offset, which the range check of
  // the buffer descriptor covers (rows past the end read as 0).
  auto dma_k = [&](uint32_t i, uint8_t* nk, uint32_t bytes) __attribute__((always_inline)) {
    uint32_t so = bytes + i * kDmaRows * k_row_bytes;
    asm volatile("" : "+s"(so));
    dma16(k_rsrc, nk + (i * kThreads + wave_s * kWave) * 16, k_voff + so);
  };
  auto dma_v = [&](uint32_t i, uint8_t* nv, uint32_t bytes) __attribute__((always_inline)) {
    uint32_t so = bytes + i * kDmaRows * v_row_bytes;
    asm volatile("" : "+s"(so));
    dma16(v_rsrc, nv + (i * kThreads + wave_s * kWave) * 16, v_voff + so);
  };

  // Software pipeline over key blocks: step j runs one MFMA cluster with the
  // scores of block j and the output update of block j - 1 (from pp), with
  // the step's DMA spread over it, then the softmax of block j on the VALU.
  // K tiles run one block ahead of V tiles: step j fetches K(j + 1) and V(j),
  // each into the stage last read in step j - 1.
  auto cluster = [&]<bool WithPv>(float16_t* s, const uint8_t* lk, const uint8_t* lv, uint8_t* nk,
                                   uint8_t* nv, uint32_t kbi) __attribute__((always_inline)) {
    const uint32_t next = kbi + 1 < nblocks ? kbi + 1 : kbi;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[st][e] = 0.0f;
    // K and V fragments two k steps ahead (four MFMAs between a fragment's
    // read and its use, which covers the LDS latency).
    constexpr uint32_t kAhead = 2;
    half8_t kf[kAhead][2], vf[kAhead][2];
    // PV MFMA n = 2 ks + st of 16: (st, h) pair n / kDT, d tile n % kDT.
    auto pv_frag = [&](uint32_t ks, uint32_t st) __attribute__((always_inline)) {
      const uint32_t n = 2 * ks + st, c = n / kDT, dt = n % kDT;
      return vfrag(lv, c / 2, c % 2, dt);
    };
#pragma unroll
    for (uint32_t ks = 0; ks < kAhead; ++ks)
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        kf[ks][st] = kfrag(lk, st, ks);
        if constexpr (WithPv) vf[ks][st] = pv_frag(ks, st);
      }
    __builtin_amdgcn_sched_barrier(0);
    // Raised priority while this wave feeds the matrix pipe: the other wave
    // on the SIMD fills the gaps with its softmax.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (uint32_t ks = 0; ks < kKS; ++ks) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        s[st] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks % kAhead][st], qf[ks], s[st], 0, 0, 0);
        if constexpr (WithPv) {
          const uint32_t n = 2 * ks + st, c = n / kDT, dt = n % kDT;
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[ks % kAhead][st], pp[c / 2][c % 2], o[dt],
                                                         0, 0, 0);
        }
      }
      if (ks + kAhead < kKS) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          kf[ks % kAhead][st] = kfrag(lk, st, ks + kAhead);
          if constexpr (WithPv) vf[ks % kAhead][st] = pv_frag(ks + kAhead, st);
        }
      }
      // DMA instructions spread over the k steps: K tile first, then V.
      constexpr uint32_t kDmaPer = (2 * KvTile<D>::kDma + kKS - 1) / kKS;
#pragma unroll
      for (uint32_t u = 0; u < kDmaPer; ++u) {
        const uint32_t i = ks * kDmaPer + u;
        if (i < KvTile<D>::kDma) dma_k(i, nk, next * k_block_bytes);
        else if (i < 2 * KvTile<D>::kDma) dma_v(i - KvTile<D>::kDma, nv, kbi * v_block_bytes);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // Output update of the previous block alone (V tile lv).
  auto pv_only = [&](const uint8_t* lv) __attribute__((always_inline)) {
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (uint32_t dt = 0; dt < kDT; ++dt)
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vfrag(lv, st, h, dt), pp[st][h], o[dt], 0, 0, 0);
  };
  // Softmax of block kbi.  s[st][r] is the score of key kb + 32 st + 8 (r/4)
  // + 4 (lane/32) + r%4 for query qi; the result goes to pp.
  auto softmax = [&](float16_t* s, uint32_t kbi) __attribute__((always_inline)) {
    const uint32_t kb = kbi * kKeysPerBlock;
    const bool need_mask = (Causal && kb + kKeysPerBlock - 1 > wq0) || kb + kKeysPerBlock > key_rows;
    if (need_mask) {
      // Key kb + 4 (lane / 32) + x is allowed iff x <= lim (the last allowed
      // key is min(qi, key_rows - 1) causal, key_rows - 1 otherwise; key_rows
      // < 2^30, so lim fits an int).
      const uint32_t last = Causal && qi < key_rows - 1 ? qi : key_rows - 1;
      const int lim = (int)last - (int)(kb + 4 * (lane / 32));
      // One compare into VCC and one select per score (compares into SGPR
      // pairs, as the compiler hoists them, run out of SGPRs).  The scores
      // come straight from MFMAs, and the hazard padding the compiler gives
      // its own VALU reads of MFMA results does not cover inline assembly:
      // 24 wait states first.
      const float ninf = -INFINITY;
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          asm volatile("v_cmp_gt_i32 vcc, %1, %2\n\tv_cndmask_b32 %0, %0, %3, vcc"
                       : "+v"(s[st][r])
                       : "n"(32 * st + 8 * (r / 4) + r % 4), "v"(lim), "v"(ninf)
                       : "vcc");
    }
    // Probabilities against the current reference point, and this lane's
    // share of the block's row sum.  The row sum adds the fp16
    // probabilities that the MFMA consumes: pairs, then quads, in fp16
    // (each p <= 2^kRescaleSlack on the accepted path, so a quad sum stays
    // far inside the fp16 range and carries at most two roundings), then
    // fp32 accumulation with v_dot2.
    auto exps = [&](float neg_m, half8_t (*pf)[2]) __attribute__((always_inline)) {
      float sum = 0.0f;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            pf[st][h][e] = (half_t)__builtin_amdgcn_exp2f(fmaf(s[st][8 * h + e], scale_log2, neg_m));
          const half2_t s01 = half2_t{pf[st][h][0], pf[st][h][1]} + half2_t{pf[st][h][2], pf[st][h][3]};
          const half2_t s45 = half2_t{pf[st][h][4], pf[st][h][5]} + half2_t{pf[st][h][6], pf[st][h][7]};
          sum = __builtin_amdgcn_fdot2(s01 + s45, half2_t{1, 1}, sum, false);
        }
      return sum;
    };
    // The reference point moves only when some probability would exceed
    // 2^kRescaleSlack, found without a max over the scores: every p is at
    // most the lane's block sum, so a block sum <= 2^kRescaleSlack accepts
    // the block (overflow to inf and NaN, as against the -inf start, fail
    // the test).  Otherwise the max of the query's 64 keys (this lane and
    // its partner lane ^ 32, so both halves share one reference point; it is
    // finite, as every processed block holds an allowed key per query)
    // becomes the reference point, the output and sum are rescaled, and the
    // probabilities are recomputed (all <= 1).  Exact for any reference
    // point.
    half8_t pf[2][2];
    float sum = exps(-m_run, pf);
    if (__any(!(sum <= kSumLimit))) {
      float mx = s[0][0];
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[st][r]);
      mx = max_with_partner(mx * scale_log2);
      const float m_new = mx > m_run ? mx : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (uint32_t dt = 0; dt < kDT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
      sum = exps(-m_run, pf);
    }
    l_run += sum;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int h = 0; h < 2; ++h) pp[st][h] = pf[st][h];
  };

  auto step = [&](const uint8_t* lk, const uint8_t* lv, uint8_t* nk, uint8_t* nv, uint32_t kbi)
      __attribute__((always_inline)) {
    // Every wave's DMA of K(kbi) and V(kbi - 1) has landed, and every wave
    // is done reading K(kbi - 1) and V(kbi - 2), whose stages the DMA of this
    // step overwrites.  The last block re-fetches its K tile: the DMA stays
    // unconditional, which keeps the compiler's wait counting exact.
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // One path for every step (separate paths for the first block and for
    // blocks past this wave's last made the compiler copy the output
    // accumulators between register sets): the first step's output MFMAs
    // add the zero probabilities pp starts with, and past the wave's last
    // block every key is masked, so the softmax yields zeros and only the
    // pending output update of the wave's last block counts.
    float16_t s[2];
    cluster.template operator()<true>(s, lk, lv, nk, nv, kbi);
    softmax(s, kbi);
  };

  // Block j lives in stage j % 2 (lds_k0 / lds_v0 for even j).  The first
  // step's output MFMAs multiply zero probabilities with V stage 1, which
  // is zeroed here (whatever an earlier kernel left in LDS may hold
  // non-finite fp16 patterns; 0 * inf is NaN).
#pragma unroll
  for (uint32_t i = 0; i < KvTile<D>::kDma; ++i) dma_k(i, lds_k0, 0);
#pragma unroll
  for (uint32_t i = 0; i < kTile / 16 / kThreads; ++i)
    *reinterpret_cast<u32x4*>(lds_v1 + (i * kThreads + threadIdx.x) * 16) = u32x4{0, 0, 0, 0};
  // Both steps of a pair run unconditionally, so the loop body is one
  // straight path (a skipped second step made the compiler merge the output
  // accumulators from two paths with register copies); an odd last block
  // runs after the loop.
  uint32_t kbi = 0;
  for (; kbi + 1 < nblocks; kbi += 2) {
    step(lds_k0, lds_v1, lds_k1, lds_v0, kbi);
    step(lds_k1, lds_v0, lds_k0, lds_v1, kbi + 1);
  }
  if (kbi < nblocks) step(lds_k0, lds_v1, lds_k1, lds_v0, kbi);
  // V of the last block (and every DMA) has landed after this barrier.
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  if (nproc == nblocks) pv_only((nblocks - 1) % 2 == 0 ? lds_v0 : lds_v1);

  // o[dt][r] = O^T[d = 32 dt + 8 (r/4) + 4 (lane/32) + r%4][qi], unnormalised.
  const float l_total = sum_with_partner(l_run);
  const float inv = 1.0f / l_total;
  if (qi < query_rows) {
    const uint64_t row = ((uint64_t)stream * query_rows + qi) * width;
#pragma unroll
    for (uint32_t dt = 0; dt < kDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t d = dt * 32 + 8 * g + 4 * (lane / 32);
        if (d >= width) continue;  // padding (width is a multiple of 8)
        if constexpr (OutF16) {
          half4_t hv;
#pragma unroll
          for (int e = 0; e < 4; ++e) hv[e] = (half_t)(o[dt][4 * g + e] * inv);
          *reinterpret_cast<half4_t*>((uint16_t*)out + row + d) = hv;
        } else {
          float4_t fv;
#pragma unroll
          for (int e = 0; e < 4; ++e) fv[e] = o[dt][4 * g + e] * inv;
          *reinterpret_cast<float4_t*>((float*)out + row + d) = fv;
        }
      }
  }
}

// One workgroup per query block (non-causal), or per pair of query blocks
// i and n - 1 - i of one stream (causal: the pair's key steps add up to the
// same count for every workgroup).  Workgroups are remapped so each XCD
// (round-robin dispatch over 8) runs whole streams, sharing K and V in its L2.
template <int D, bool Causal, bool OutF16>
__global__ __launch_bounds__(kThreads, 2) void attention_fwd_kernel(
    void* __restrict__ out, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, uint32_t streams, uint32_t query_rows, uint32_t key_rows,
    uint32_t width, float scale_log2, uint32_t q_heads, uint32_t k_heads, uint32_t v_heads) {
  const uint32_t qblocks = (query_rows + kQueriesPerBlock - 1) / kQueriesPerBlock;
  const uint32_t per_stream = Causal ? (qblocks + 1) / 2 : qblocks;
  const uint32_t total = per_stream * streams;
  uint32_t pid = blockIdx.x;
  if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;  // XCD-contiguous
  const uint32_t stream = pid / per_stream, i = pid % per_stream;
  // Causal: the heavy block first, then its mirror (none for the middle
  // block of an odd count).
  const uint32_t reps = Causal && i != qblocks - 1 - i ? 2 : 1;
  for (uint32_t rep = 0; rep < reps; ++rep) {
    // Every wave is done with the LDS stages before the next block's DMA.
    if (rep > 0) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const uint32_t qb = Causal ? (rep == 0 ? qblocks - 1 - i : i) : i;
    attention_block<D, Causal, OutF16>(out, query, key, value, stream, qb, query_rows, key_rows,
                                       width, scale_log2, q_heads, k_heads, v_heads);
  }
}

// General attention: one 64-lane block per (stream, query row); any widths.
// Online softmax over keys one at a time (dot products by wave reduction).
constexpr uint32_t kGeneralMaxValuePerLane = 8;  // value width <= 512

__global__ __launch_bounds__(64) void attention_general_kernel(
    void* __restrict__ out, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, uint32_t query_rows, uint32_t key_rows, uint32_t width,
    uint32_t value_width, float scale_log2, bool causal, bool out_f16, uint32_t q_heads,
    uint32_t k_heads, uint32_t v_heads) {
  const uint64_t flat = blockIdx.x;
  const uint32_t stream = (uint32_t)(flat / query_rows);
  const uint32_t row = (uint32_t)(flat % query_rows);
  const uint32_t lane = threadIdx.x;
  // Head layout as in the fast kernel; K and V rows are k_pitch / v_pitch apart.
  const uint16_t* q = query + (((uint64_t)(stream / q_heads) * query_rows + row) * q_heads +
                               stream % q_heads) * width;
  const uint64_t k_pitch = (uint64_t)k_heads * width, v_pitch = (uint64_t)v_heads * value_width;
  const uint16_t* K = key + (uint64_t)(stream / k_heads) * key_rows * k_pitch + (stream % k_heads) * width;
  const uint16_t* V = value + (uint64_t)(stream / v_heads) * key_rows * v_pitch +
                      (stream % v_heads) * value_width;
  uint32_t allowed = key_rows;
  if (causal) allowed = row + 1 < key_rows ? row + 1 : key_rows;
  float acc[kGeneralMaxValuePerLane];
#pragma unroll
  for (uint32_t i = 0; i < kGeneralMaxValuePerLane; ++i) acc[i] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  for (uint32_t j = 0; j < allowed; ++j) {
    float dot = 0.0f;
    for (uint32_t d = lane; d < width; d += 64)
      dot += (float)__builtin_bit_cast(half_t, q[d]) *
             (float)__builtin_bit_cast(half_t, K[(uint64_t)j * k_pitch + d]);
    dot = wave_sum(dot) * scale_log2;
    const float m_new = fmaxf(m, dot);
    const float alpha = exp2f(m - m_new);
    const float p = exp2f(dot - m_new);
    l = l * alpha + p;
#pragma unroll
    for (uint32_t i = 0; i < kGeneralMaxValuePerLane; ++i) {
      const uint32_t c = lane + 64 * i;
      const float v = c < value_width ? (float)__builtin_bit_cast(half_t, V[(uint64_t)j * v_pitch + c]) : 0.0f;
      acc[i] = acc[i] * alpha + p * v;
    }
    m = m_new;
  }
  const float inv = 1.0f / l;
#pragma unroll
  for (uint32_t i = 0; i < kGeneralMaxValuePerLane; ++i) {
    const uint32_t c = lane + 64 * i;
    if (c < value_width) {
      const float r = acc[i] * inv;
      if (out_f16)
        ((uint16_t*)out)[flat * value_width + c] = __builtin_bit_cast(uint16_t, (half_t)r);
      else
        ((float*)out)[flat * value_width + c] = r;
    }
  }
}

template <int D, bool Causal, bool OutF16>
int launch_fast(hipStream_t stream, const AttentionArgs& a, float scale_log2) {
  const uint32_t qblocks = (a.query_rows + kQueriesPerBlock - 1) / kQueriesPerBlock;
  const uint64_t blocks = (uint64_t)(Causal ? (qblocks + 1) / 2 : qblocks) * a.streams;
  if (blocks > 0x7fffffffu) return IPUS_ERROR_INVALID_ARGUMENT;
  hipLaunchKernelGGL((attention_fwd_kernel<D, Causal, OutF16>), dim3((uint32_t)blocks),
                     dim3(kThreads), 0, stream, a.out, (const uint16_t*)a.query,
                     (const uint16_t*)a.key, (const uint16_t*)a.value, a.streams, a.query_rows,
                     a.key_rows, a.width, scale_log2, a.heads[0], a.heads[1], a.heads[2]);
  return hip_status(hipGetLastError());
}

template <int D>
int dispatch_fast(hipStream_t stream, const AttentionArgs& a, float scale_log2) {
  if (a.causal)
    return a.output_f16 ? launch_fast<D, true, true>(stream, a, scale_log2)
                        : launch_fast<D, true, false>(stream, a, scale_log2);
  return a.output_f16 ? launch_fast<D, false, true>(stream, a, scale_log2)
                      : launch_fast<D, false, false>(stream, a, scale_log2);
}

}  // namespace

int launch_attention_f16(hipStream_t stream, const AttentionArgs& a) {
  if (a.streams == 0 || a.query_rows == 0) return 0;
  if (a.key_rows == 0 || a.width == 0 || a.value_width == 0) return IPUS_ERROR_INVALID_ARGUMENT;
  if (!(a.scale > 0.0f) || a.scale == INFINITY) return IPUS_ERROR_INVALID_ARGUMENT;
  const float scale_log2 = a.scale * kLog2e;
  const bool aligned = ((uintptr_t)a.query % 16 == 0) && ((uintptr_t)a.key % 16 == 0) &&
                       ((uintptr_t)a.value % 16 == 0) && ((uintptr_t)a.out % 16 == 0);
  for (int i = 0; i < 3; ++i)
    if (a.heads[i] == 0 || a.streams % a.heads[i] != 0) return IPUS_ERROR_INVALID_ARGUMENT;
  // The fast kernel addresses one stream's K or V through a buffer
  // descriptor with a 31-bit byte range; the offsets of the last block's
  // rows (up to 63 past the end) and of padding chunks stay below 2^32.
  const uint64_t kv_pitch = (uint64_t)(a.heads[1] > a.heads[2] ? a.heads[1] : a.heads[2]) * a.width * 2;
  const bool fits = ((uint64_t)a.key_rows + kKeysPerBlock) * kv_pitch <= 0x7fff0000ull;
  // Widths that are multiples of 8 up to 128 run in 64- or 128-wide tiles
  // (zero padding); others take the general kernel.
  if (aligned && fits && a.width == a.value_width && a.width % 8 == 0 && a.width <= 128) {
    return a.width > 64 ? dispatch_fast<128>(stream, a, scale_log2)
                        : dispatch_fast<64>(stream, a, scale_log2);
  }
  if (a.value_width > 64 * kGeneralMaxValuePerLane) return IPUS_ERROR_UNAVAILABLE;
  const uint64_t blocks = (uint64_t)a.streams * a.query_rows;
  if (blocks > 0x7fffffffu) return IPUS_ERROR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(attention_general_kernel, dim3((uint32_t)blocks), dim3(64), 0, stream, a.out,
                     (const uint16_t*)a.query, (const uint16_t*)a.key, (const uint16_t*)a.value,
                     a.query_rows, a.key_rows, a.width, a.value_width, scale_log2, a.causal,
                     a.output_f16, a.heads[0], a.heads[1], a.heads[2]);
  return hip_status(hipGetLastError());
}

}  // namespace ipus
