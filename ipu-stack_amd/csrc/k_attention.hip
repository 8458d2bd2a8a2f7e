// Fused online-softmax attention on gfx950 MFMA:
//   O = softmax(scale * Q K^T [+ causal mask]) V
// Q, K, V fp16 [streams, rows, width]; fp32 scores, running max and sum;
// fp32 output by default (the reference's device attention output precision,
// crates/ipu-codegen/src/mid.rs:2064-2067) or fp16.  Semantics:
// device/flash_attention_online_f16.cpp:68-143 (online softmax, exact) and
// crates/ipu-tests/src/diagnostic.rs:711-780 (key j allowed iff j <= i when
// causal, 741-745; scale default 1/sqrt(width), 733-736).
//
// Fast kernel (query/key and value widths multiples of 8 up to 256, equal
// or with tiles 128/64, 64/128, 256/128 or 128/256; stored in LDS tiles 64,
// 128 or 256 columns wide with zero padding; for equal widths the MFMAs
// cover the width rounded up to 32 columns):
//   * 256 threads = 4 waves; a wave owns 32 queries (two tiles of 16; one
//     tile at 256 columns), a workgroup 128 (64) queries of one stream; two
//     workgroups share a CU (launch bound), so one SIMD runs the softmax of
//     one wave while the MFMA pipe serves the other;
//   * keys stream through LDS in blocks of 64 (32 at 256 columns) with two
//     stages.  K and V tiles are copied global -> LDS with buffer_load ...
//     lds (16 bytes per lane, no staging registers; rows past the end of the
//     stream read as 0), both stored row-major [keys][D] with an XOR swizzle
//     of 16-byte chunks;
//   * v_mfma_f32_16x16x32_f16 throughout: under the board's power limit it
//     sustains a higher clock than 32 x 32 x 16 on changing operands;
//   * software pipeline: step j runs ONE MFMA cluster holding the scores of
//     block j and the output update of block j - 1 (alternating, fragments
//     read ahead, the step's DMA instructions spread between them), then the
//     softmax of block j on the VALU.  K tiles run one block ahead of V;
//   * scores are computed transposed, S^T = K Q^T (K fragments by
//     ds_read_b128 as the first operand, Q fragments resident in registers
//     as the second), so a lane holds 4 consecutive keys of one query per
//     16 x 16 tile: four lanes share a query, whose max needs two exchanges
//     and whose running sum none until the end;
//   * the output is accumulated transposed, O^T += V^T P^T: the fp16
//     probabilities are the second MFMA operand straight from the score
//     registers, and the matching V^T fragments come from the row-major V
//     tile through ds_read_b64_tr_b16, whose 4-key runs are chosen to follow
//     the score accumulator's key order;
//   * each fragment read feeds one MFMA per query tile of the wave;
//   * the reference point (running max) moves only when some probability of
//     a block would exceed kSumLimit (2^8), which the block's probability
//     sum bounds, so no max over the scores is taken on the common path:
//     the result is exact for any reference point, and most blocks skip the
//     max, the rescale of the output accumulators and the lane exchanges;
//   * K and V fragment offsets are computed once per lane (XOR swizzles of
//     one base), so the cluster's LDS reads take immediate offsets only;
//   * causal: key blocks past the workgroup's last query are never loaded, a
//     wave skips blocks past its own last query.
//   * a workgroup runs two query blocks of one stream back to back (causal:
//     n - 1 - i and then i, so every workgroup has the same number of key
//     steps); the first block's last step prefetches the second's first K
//     tile and Q fragments;
//     workgroups are remapped so each XCD (round-robin dispatch over 8) runs
//     whole streams, sharing K and V in its L2.
#include "../../include/ipus.h"
#include "device_common.h"
#include "kernels.h"

#define LDS_AS __attribute__((address_space(3)))

namespace ipus {
namespace {

constexpr int kThreads = 256;
// Fast-kernel shape for tile width D: 16-query tiles per wave and keys per
// block.  Up to 128 columns a wave owns two query tiles (32 queries) and a
// block is 64 keys; at 256 columns one tile and 32 keys keep the registers
// (output accumulators, Q fragments) within two waves per SIMD and the two
// LDS stages within two workgroups per CU.
template <int D>
struct Fast {
  static constexpr int kQT = D > 128 ? 1 : 2;           // 16-query tiles per wave
  static constexpr int kKeys = D > 128 ? 32 : 64;       // keys per block
  static constexpr int kQueriesPerWave = 16 * kQT;
  static constexpr int kQueriesPerBlock = 4 * kQueriesPerWave;  // per workgroup
  static constexpr int kKT = kKeys / 16;                // 16-key score tiles per block
  static constexpr int kHalves = kKeys / 32;            // 32-key output contractions per block
};
constexpr int kMaxKeysPerBlock = 64;
constexpr uint32_t kBlocksPerGroup = 2;  // query blocks per workgroup, run back to back
constexpr float kLog2e = 1.4426950408889634f;
// A block whose probabilities, taken against the current reference point,
// sum to at most 2^8 per lane is accepted without moving the reference.
constexpr float kSumLimit = 256.0f;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, dword 3 of the descriptor

typedef short short4_t __attribute__((vector_size(8)));

inline int hip_status(hipError_t e) { return e == hipSuccess ? 0 : IPUS_ERROR_HIP_BASE - (int)e; }

// Tiles of Fast<D>::kKeys keys x D fp16, rows of D * 2 bytes, 16-byte
// chunks swizzled by row.  K is read with ds_read_b128 (each 16-lane group:
// 16 consecutive rows of one chunk), V with ds_read_b64_tr_b16 (each 16-lane
// group: 4 consecutive rows x 32 bytes, 16 consecutive rows per
// instruction).  The XORs below read both without bank conflicts
// (SQ_LDS_BANK_CONFLICT = 0 in a probe of the two patterns on 128- and
// 256-byte rows).  They depend only on the row's low bits and change only
// the low 4 bits of the chunk index, and a bank is fixed by the byte offset
// modulo 256, so 512-byte rows (D = 256) see the 256-byte rows' pattern.
template <int D, int Keys>
struct KvTile {
  static constexpr uint32_t kRowBytes = D * 2;
  static constexpr uint32_t kChunks = D / 8;
  static constexpr uint32_t kBytes = Keys * D * 2;
  static constexpr uint32_t kDma = kBytes / 16 / kThreads;  // DMA instructions per thread
  static constexpr uint32_t kDmaRows = kThreads / kChunks;   // rows per DMA instruction
};
template <int D>
__device__ __forceinline__ uint32_t k_swz(uint32_t row) {
  return D >= 128 ? (row & 15u) : (row & 7u);
}
template <int D>
__device__ __forceinline__ uint32_t v_swz(uint32_t row) {
  return D >= 128 ? ((row & 7u) << 1) : (row & 7u);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// max / sum of x over the four lanes l ^ {0, 16, 32, 48} that hold one query.
__device__ __forceinline__ float max_of_query(float x) {
  x = fmaxf(x, __shfl_xor(x, 16, kWave));
  return fmaxf(x, __shfl_xor(x, 32, kWave));
}
__device__ __forceinline__ float sum_of_query(float x) {
  x += __shfl_xor(x, 16, kWave);
  return x + __shfl_xor(x, 32, kWave);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LDS_AS void*)lds, 16, voffset, 0, 0, 0);
}

// Byte offset within a key block of the chunk this thread's first DMA
// instruction fetches: instruction i of thread t fills LDS slot i * 256 + t,
// so it loads the chunk that the swizzle places there.  Instruction i covers
// the rows kThreads / kChunks * i further on; the other instructions add a
// wave-uniform row offset.  The swizzles depend on row bits 0-3 (K at D >=
// 128) or 0-2, which a step of 16 or 32 rows leaves alone; at D = 256 a step
// is 8 rows, so the odd instructions' K chunks are those of row + 8
// (first_row = 8), the even ones' those of row.  row_bytes is the global row
// pitch: width * 2 for a contiguous [streams, rows, width] tensor, heads *
// width * 2 for a head of an unsplit [batch, rows, heads * width].  Chunks at
// or past the width (a width below the tile's D, padded) get an offset past
// the buffer's range, so their loads return 0: kPadOffset plus any block
// offset (< 2^31) stays above the range (< 0x7fff0000) without wrapping.
constexpr uint32_t kPadOffset = 0x80000000u;
template <int D, bool IsK>
__device__ __forceinline__ uint32_t kv_offset(uint32_t row_bytes, uint32_t width,
                                              uint32_t first_row = 0) {
  const uint32_t row = threadIdx.x / (D / 8), phys = threadIdx.x % (D / 8);
  const uint32_t srow = row + first_row;
  const uint32_t chunk = phys ^ (IsK ? k_swz<D>(srow) : v_swz<D>(srow));
  return chunk * 8 < width ? row * row_bytes + chunk * 16 : kPadOffset;
}

// Key blocks of query block qb: causal blocks stop at the block's last query.
template <int D, bool Causal>
__device__ __forceinline__ uint32_t key_blocks(uint32_t qb, uint32_t query_rows, uint32_t key_rows) {
  constexpr uint32_t kQPB = Fast<D>::kQueriesPerBlock, kKeys = Fast<D>::kKeys;
  uint32_t key_end = key_rows;
  if (Causal) {
    const uint32_t q0 = qb * kQPB;
    const uint32_t last_q = q0 + kQPB < query_rows ? q0 + kQPB : query_rows;
    key_end = last_q < key_rows ? last_q : key_rows;
  }
  return (key_end + kKeys - 1) / kKeys;
}

// The wave's Q fragments for query block qb (second MFMA operand of the
// scores): tile qt, k step ks holds Q[query][32 ks + 8 (l / 16) .. +7] of
// query qb * kQueriesPerBlock + wave * kQueriesPerWave + 16 qt + l % 16
// (clamped to the last row; padding columns are 0).
template <int D, int DC>
__device__ __forceinline__ void load_q(half8_t (&qf)[Fast<D>::kQT][DC / 32], const uint16_t* __restrict__ query,
                                       uint32_t stream, uint32_t qb, uint32_t query_rows,
                                       uint32_t width, uint32_t q_heads) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t r16 = lane % 16, g4 = lane / 16;
  const uint32_t wave_s = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t wq0 = qb * Fast<D>::kQueriesPerBlock + wave_s * Fast<D>::kQueriesPerWave;
  const uint32_t q_pitch = q_heads * width;
  const uint16_t* Q = query + (uint64_t)(stream / q_heads) * query_rows * q_pitch + (stream % q_heads) * width;
#pragma unroll
  for (uint32_t qt = 0; qt < Fast<D>::kQT; ++qt) {
    uint32_t q = wq0 + 16 * qt + r16;
    q = q < query_rows ? q : query_rows - 1;
#pragma unroll
    for (uint32_t ks = 0; ks < DC / 32; ++ks) {
      const uint32_t d0 = ks * 32 + g4 * 8;
      qf[qt][ks] = __builtin_bit_cast(
          half8_t, d0 < width ? load16(Q + (uint64_t)q * q_pitch + d0) : u32x4{0, 0, 0, 0});
    }
  }
}

// D / DC: K tile width and score columns (query/key width); DV / DVC: V
// tile width and output columns (value width).  The block shape (query
// tiles per wave, keys per block) follows the wider tile.
template <int D, int DC, int DV, int DVC, bool Causal, bool OutF16>
__device__ __forceinline__ void attention_block(
    void* __restrict__ out, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, uint32_t stream, uint32_t qb, uint32_t query_rows,
    uint32_t key_rows, uint32_t width, uint32_t value_width, float scale_log2, uint32_t q_heads,
    uint32_t k_heads, uint32_t v_heads, half8_t (&qf)[Fast<(D > DV ? D : DV)>::kQT][DC / 32],
    bool k0_loaded, bool chain, uint32_t next_qb) {
  using F = Fast<(D > DV ? D : DV)>;
  constexpr int kQT = F::kQT, kKT = F::kKT, kHalves = F::kHalves;
  constexpr uint32_t kKeys = F::kKeys;
  constexpr uint32_t kQPW = F::kQueriesPerWave, kQPB = F::kQueriesPerBlock;
  static_assert(DC % 32 == 0 && DC <= D, "score columns: whole k steps of the tile");
  static_assert(DVC % 16 == 0 && DVC <= DV, "output columns: whole d tiles of the tile");
  constexpr uint32_t kKS = DC / 32;   // k steps (32 columns) of the score MFMAs
  constexpr uint32_t kDT = DVC / 16;  // output d tiles (16 columns)
  constexpr uint32_t kScoreGroups = kKT * kKS;   // score MFMA groups (every query tile) per block
  constexpr uint32_t kOutGroups = kHalves * kDT;  // output MFMA groups per block
  constexpr uint32_t kPairs = kScoreGroups > kOutGroups ? kScoreGroups : kOutGroups;
  using KT = KvTile<D, kKeys>;
  using VT = KvTile<DV, kKeys>;
  constexpr uint32_t kRB = KT::kRowBytes, kVRB = VT::kRowBytes;
  constexpr uint32_t kTile = KT::kBytes, kVTile = VT::kBytes;
  constexpr uint32_t kDmaRows = KT::kDmaRows, kVDmaRows = VT::kDmaRows;
  // Two stages, each a distinct LDS object so the compiler can see that the
  // DMA into one stage never aliases the fragment reads of the other.
  __shared__ __attribute__((aligned(1024))) uint8_t lds_k0[kTile];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_v0[kVTile];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_k1[kTile];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_v1[kVTile];

  const uint32_t q0 = qb * kQPB;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t r16 = lane % 16, g4 = lane / 16;
  const uint32_t wave_s = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const uint32_t wq0 = q0 + wave_s * kQPW;  // first query of this wave

  // Stream s of an operand with h heads is head s % h of matrix s / h of a
  // [streams / h, rows, h * w] tensor (h = 1: contiguous [streams, rows, w];
  // w the operand's width).  The tile widths are the widths padded to 64,
  // 128 or 256.
  const uint32_t k_row_bytes = k_heads * width * 2u, v_row_bytes = v_heads * value_width * 2u;
  const uint16_t* K = key + (uint64_t)(stream / k_heads) * key_rows * k_heads * width + (stream % k_heads) * width;
  const uint16_t* V = value + (uint64_t)(stream / v_heads) * key_rows * v_heads * value_width +
                      (stream % v_heads) * value_width;
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)K, 0, (int)((key_rows - 1) * k_row_bytes + width * 2u), kBufferFlags);
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)V, 0, (int)((key_rows - 1) * v_row_bytes + value_width * 2u), kBufferFlags);
  // K chunks of even and odd DMA instructions (they differ only at D = 256).
  const uint32_t k_voff = kv_offset<D, true>(k_row_bytes, width);
  const uint32_t k_voff_odd = kDmaRows % 16 == 0 ? k_voff : kv_offset<D, true>(k_row_bytes, width, kDmaRows);
  const uint32_t v_voff = kv_offset<DV, false>(v_row_bytes, value_width);
  static_assert(kVDmaRows % 8 == 0, "the V swizzle depends on row bits 0-2 only");

  const uint32_t nblocks = key_blocks<(D > DV ? D : DV), Causal>(qb, query_rows, key_rows);
  const uint32_t k_block_bytes = kKeys * k_row_bytes;
  const uint32_t v_block_bytes = kKeys * v_row_bytes;
  // Blocks this wave computes scores for (causal: keys <= its last query).
  // Every such block holds at least one allowed key per query of the wave.
  uint32_t nproc = nblocks;
  if (Causal) {
    const uint32_t lim = (wq0 + kQPW - 1) / kKeys + 1;
    nproc = lim < nproc ? lim : nproc;
  }

  float4_t o[kDT][kQT];
#pragma unroll
  for (uint32_t dt = 0; dt < kDT; ++dt)
#pragma unroll
    for (uint32_t qt = 0; qt < kQT; ++qt) o[dt][qt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run[kQT];  // reference points, log2 units (scaled)
  float l_run[kQT];  // this lane's share of the row sums
  uint32_t qi[kQT];  // this lane's query in tile qt
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.0f;
    qi[qt] = wq0 + 16 * qt + r16;
  }
  half8_t pp[kHalves][kQT];  // fp16 probabilities of the last softmax [key half kk][qt]
#pragma unroll
  for (int kk = 0; kk < kHalves; ++kk)
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt)
#pragma unroll
      for (int e = 0; e < 8; ++e) pp[kk][qt][e] = (half_t)0.0f;  // "block -1"

  // Score accumulator s[kt][qt] (v_mfma_f32_16x16x32_f16 of K tile kt as the
  // first operand): element e is key 16 kt + 4 (l / 16) + e of query qt.
  // Output MFMAs contract 32 keys (half kk of the block): k slot 8 (l / 16) + e
  // is key 32 kk + 4 (l / 16) + e for e < 4 and 32 kk + 16 + 4 (l / 16) + e - 4
  // otherwise, which is how pp packs the score elements, so each lane's
  // probabilities feed the MFMA where they are.
  // K fragment for key tile kt, k step ks: lane holds K[16 kt + l % 16][32 ks
  // + 8 (l / 16) .. +7] (ds_read_b128).  V^T fragment for d tile dt and half
  // kk: lane holds d = 16 dt + l % 16 of the 8 keys of its k slots, two
  // ds_read_b64_tr_b16 of 4 consecutive keys each (in a 16-lane group, source
  // lane s addresses key k0 + s / 4, columns 16 dt + 4 (s % 4) .. +3).  The
  // swizzles depend on the row's low bits only, so the offsets are per-lane
  // bases XORed with the k step or d tile plus an immediate row offset.
  const uint32_t kbase = r16 * kRB + ((g4 ^ k_swz<D>(r16)) << 4);
  uint32_t vbase;
  {
    const uint32_t row = 4 * g4 + r16 / 4, c1 = (r16 % 4) / 2;
    vbase = row * kVRB + ((c1 ^ v_swz<DV>(row)) << 4) + 8 * (r16 % 2);
  }
  uint32_t kofs[kKS], vofs[kDT];
#pragma unroll
  for (uint32_t ks = 0; ks < kKS; ++ks) kofs[ks] = kbase ^ (ks << 6);
#pragma unroll
  for (uint32_t dt = 0; dt < kDT; ++dt) vofs[dt] = vbase ^ (dt << 5);
  auto kfrag = [&](const uint8_t* lk, uint32_t kt, uint32_t ks) __attribute__((always_inline)) {
    const uint8_t* p = lk + kofs[ks] + 16 * kt * kRB;
    return __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4*>(p));
  };
  auto vfrag = [&](const uint8_t* lv, uint32_t dt, uint32_t kk) __attribute__((always_inline)) {
    const uint8_t* p = lv + vofs[dt] + 32 * kk * kVRB;
    const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)p);
    const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)(p + 16 * kVRB));
    return __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  // DMA instruction i of a K or V tile.  The scalar part is opaque so the
  // per-instruction offsets are not hoisted out of the loop into registers;
  // the block offset stays in the vector offset, which the range check of
  // the buffer descriptor covers (rows past the end read as 0).
  auto dma_k = [&](uint32_t i, uint8_t* nk, uint32_t bytes) __attribute__((always_inline)) {
    uint32_t so = bytes + i * kDmaRows * k_row_bytes;
    asm volatile("" : "+s"(so));
    dma16(k_rsrc, nk + (i * kThreads + wave_s * kWave) * 16, (i % 2 ? k_voff_odd : k_voff) + so);
  };
  auto dma_v = [&](uint32_t i, uint8_t* nv, uint32_t bytes) __attribute__((always_inline)) {
    uint32_t so = bytes + i * kVDmaRows * v_row_bytes;
    asm volatile("" : "+s"(so));
    dma16(v_rsrc, nv + (i * kThreads + wave_s * kWave) * 16, v_voff + so);
  };

  // Software pipeline over key blocks: step j runs one MFMA cluster with the
  // scores of block j and the output update of block j - 1 (from pp), with
  // the step's DMA spread over it, then the softmax of block j on the VALU.
  // K tiles run one block ahead of V tiles: step j fetches K(j + 1) and V(j),
  // each into the stage last read in step j - 1.  Pair p of the cluster is
  // score pair (k step p / 4, key tile p % 4) and output pair (half p / kDT,
  // d tile p % kDT), each over query tiles 0 and 1 with one fragment read.
  auto cluster = [&]<bool WithPv>(float4_t (*s)[kQT], const uint8_t* lk, const uint8_t* lv, uint8_t* nk,
                                   uint8_t* nv, uint32_t kbi) __attribute__((always_inline)) {
    const uint32_t next = kbi + 1 < nblocks ? kbi + 1 : (chain ? 0u : kbi);
#pragma unroll
    for (int kt = 0; kt < kKT; ++kt)
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) s[kt][qt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // Fragments two groups ahead (one for the 96-column tiles, which spill
    // past 256 registers with two).
    constexpr uint32_t kAhead = kQT == 2 && kKS == 3 ? 1 : 2;
    half8_t kf[kAhead], vf[kAhead];
#pragma unroll
    for (uint32_t p = 0; p < kAhead; ++p) {
      if (p < kScoreGroups) kf[p] = kfrag(lk, p % kKT, p / kKT);
      if constexpr (WithPv)
        if (p < kOutGroups) vf[p] = vfrag(lv, p % kDT, p / kDT);
    }
    __builtin_amdgcn_sched_barrier(0);
    // Raised priority while this wave feeds the matrix pipe: the other wave
    // on the SIMD fills the gaps with its softmax.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (uint32_t p = 0; p < kPairs; ++p) {
      const uint32_t ks = p / kKT, kt = p % kKT, kk = p / kDT, dt = p % kDT;
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        if (p < kScoreGroups)
          s[kt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[p % kAhead], qf[qt][ks], s[kt][qt], 0, 0, 0);
        if constexpr (WithPv)
          if (p < kOutGroups)
            o[dt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[p % kAhead], pp[kk][qt], o[dt][qt], 0, 0, 0);
      }
      if (p + kAhead < kScoreGroups) kf[p % kAhead] = kfrag(lk, (p + kAhead) % kKT, (p + kAhead) / kKT);
      if constexpr (WithPv)
        if (p + kAhead < kOutGroups) vf[p % kAhead] = vfrag(lv, (p + kAhead) % kDT, (p + kAhead) / kDT);
      // DMA instructions spread over the groups: K tile first, then V.
      constexpr uint32_t kDmaPer = (KT::kDma + VT::kDma + kPairs - 1) / kPairs;
#pragma unroll
      for (uint32_t u = 0; u < kDmaPer; ++u) {
        const uint32_t i = p * kDmaPer + u;
        if (i < KT::kDma) dma_k(i, nk, next * k_block_bytes);
        else if (i < KT::kDma + VT::kDma) dma_v(i - KT::kDma, nv, kbi * v_block_bytes);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // Output update of the previous block alone (V tile lv).
  auto pv_only = [&](const uint8_t* lv) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t kk = 0; kk < kHalves; ++kk)
#pragma unroll
      for (uint32_t dt = 0; dt < kDT; ++dt) {
        const half8_t v = vfrag(lv, dt, kk);
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
          o[dt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v, pp[kk][qt], o[dt][qt], 0, 0, 0);
      }
  };
  // Softmax of block kbi.  s[kt][qt][e] is the score of key kb + 16 kt +
  // 4 (l / 16) + e for query qi[qt]; the result goes to pp.
  auto softmax = [&](float4_t (*s)[kQT], uint32_t kbi) __attribute__((always_inline)) {
    const uint32_t kb = kbi * kKeys;
    const bool need_mask = (Causal && kb + kKeys - 1 > wq0) || kb + kKeys > key_rows;
    if (need_mask) {
      // Key kb + 4 (l / 16) + x is allowed for query qi iff x <= lim (the
      // last allowed key is min(qi, key_rows - 1) causal, key_rows - 1
      // otherwise; key_rows < 2^30, so lim fits an int).  One compare into
      // VCC and one select per score; the scores come straight from MFMAs,
      // and the hazard padding the compiler gives its own VALU reads of MFMA
      // results does not cover inline assembly: 24 wait states first.
      int lim[kQT];
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        const uint32_t last = Causal && qi[qt] < key_rows - 1 ? qi[qt] : key_rows - 1;
        lim[qt] = (int)last - (int)(kb + 4 * g4);
      }
      const float ninf = -INFINITY;
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
      for (int kt = 0; kt < kKT; ++kt)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            asm volatile("v_cmp_gt_i32 vcc, %1, %2\n\tv_cndmask_b32 %0, %0, %3, vcc"
                         : "+v"(s[kt][qt][e])
                         : "n"(16 * kt + e), "v"(lim[qt]), "v"(ninf)
                         : "vcc");
    }
    // Probabilities against the current reference points, and this lane's
    // share of each query's block sum: the fp16 probabilities that the MFMA
    // consumes, added in pairs and quads in fp16 (each p <= kSumLimit (2^8)
    // on the accepted path, so a quad sum stays far inside the fp16 range
    // and carries at most two roundings), then accumulated in fp32 by v_dot2.
    auto exps = [&](const float* neg_m, half8_t (*pf)[kQT], float* sum) __attribute__((always_inline)) {
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        sum[qt] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < kHalves; ++kk) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            pf[kk][qt][e] = (half_t)__builtin_amdgcn_exp2f(
                fmaf(s[2 * kk + e / 4][qt][e % 4], scale_log2, neg_m[qt]));
          const half2_t s01 = half2_t{pf[kk][qt][0], pf[kk][qt][1]} + half2_t{pf[kk][qt][2], pf[kk][qt][3]};
          const half2_t s45 = half2_t{pf[kk][qt][4], pf[kk][qt][5]} + half2_t{pf[kk][qt][6], pf[kk][qt][7]};
          sum[qt] = __builtin_amdgcn_fdot2(s01 + s45, half2_t{1, 1}, sum[qt], false);
        }
      }
    };
    // A reference point moves only when some probability would exceed
    // kSumLimit (2^8), found without a max over the scores: every p is at
    // most its lane's block sum, so sums <= kSumLimit (2^8) accept the block
    // (overflow to inf and NaN, as against the -inf start, fail the test).
    // Otherwise each query's max over the block's keys (the four lanes that hold
    // it, so they share one reference point; finite, as every processed block
    // holds an allowed key per query) becomes its reference point, the
    // output and sum are rescaled, and the probabilities recomputed (all
    // <= 1).  Exact for any reference point.
    half8_t pf[kHalves][kQT];
    float sum[kQT], neg_m[kQT];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) neg_m[qt] = -m_run[qt];
    exps(neg_m, pf, sum);
    bool over = false;
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) over = over || !(sum[qt] <= kSumLimit);
    if (__any(over)) {
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        float mx = s[0][qt][0];
#pragma unroll
        for (int kt = 0; kt < kKT; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) mx = fmaxf(mx, s[kt][qt][e]);
        mx = max_of_query(mx * scale_log2);
        const float m_new = mx > m_run[qt] ? mx : m_run[qt];
        const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
        m_run[qt] = m_new;
        neg_m[qt] = -m_new;
        l_run[qt] *= alpha;
#pragma unroll
        for (uint32_t dt = 0; dt < kDT; ++dt) o[dt][qt] *= alpha;
      }
      exps(neg_m, pf, sum);
    }
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) l_run[qt] += sum[qt];
#pragma unroll
    for (int kk = 0; kk < kHalves; ++kk)
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) pp[kk][qt] = pf[kk][qt];
  };

  auto step = [&](const uint8_t* lk, const uint8_t* lv, uint8_t* nk, uint8_t* nv, uint32_t kbi)
      __attribute__((always_inline)) {
    // Every wave's DMA of K(kbi) and V(kbi - 1) has landed, and every wave
    // is done reading K(kbi - 1) and V(kbi - 2), whose stages the DMA of this
    // step overwrites.  The last block re-fetches its K tile: the DMA stays
    // unconditional, which keeps the compiler's wait counting exact.
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // One path for every step: the first step's output MFMAs add the zero
    // probabilities pp starts with, and past the wave's last block every key
    // is masked, so the softmax yields zeros and only the pending output
    // update of the wave's last block counts.
    float4_t s[kKT][kQT];
    cluster.template operator()<true>(s, lk, lv, nk, nv, kbi);
    softmax(s, kbi);
  };

  // Block j lives in stage j % 2 (lds_k0 / lds_v0 for even j); K(0) is
  // fetched here unless the previous block's last step already did.  The
  // first step's output MFMAs multiply zero probabilities with V stage 1,
  // which is zeroed here (whatever an earlier kernel or block left in LDS
  // may hold non-finite fp16 patterns; 0 * inf is NaN).  With a chained
  // next block, its Q fragments are loaded once this block's last scores
  // are done with them.
#pragma unroll
  for (uint32_t i = 0; i < KT::kDma; ++i)
    if (!k0_loaded) dma_k(i, lds_k0, 0);
#pragma unroll
  for (uint32_t i = 0; i < kVTile / 16 / kThreads; ++i)
    *reinterpret_cast<u32x4*>(lds_v1 + (i * kThreads + threadIdx.x) * 16) = u32x4{0, 0, 0, 0};
  // Both steps of a pair run unconditionally, so the loop body is one
  // straight path; an odd last block runs after the loop.
  uint32_t kbi = 0;
  for (; kbi + 1 < nblocks; kbi += 2) {
    step(lds_k0, lds_v1, lds_k1, lds_v0, kbi);
    step(lds_k1, lds_v0, lds_k0, lds_v1, kbi + 1);
  }
  if (kbi < nblocks) step(lds_k0, lds_v1, lds_k1, lds_v0, kbi);
  // V of the last block (and every DMA) has landed after this barrier.
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  if (chain) load_q<(D > DV ? D : DV), DC>(qf, query, stream, next_qb, query_rows, width, q_heads);
  if (nproc == nblocks) pv_only((nblocks - 1) % 2 == 0 ? lds_v0 : lds_v1);

  // o[dt][qt][e] = O^T[d = 16 dt + 4 (l / 16) + e][qi[qt]], unnormalised.
  if constexpr (OutF16) {
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      const float inv = 1.0f / sum_of_query(l_run[qt]);
      if (qi[qt] < query_rows) {
        const uint64_t row = ((uint64_t)stream * query_rows + qi[qt]) * value_width;
#pragma unroll
        for (uint32_t dt = 0; dt < kDT; ++dt) {
          const uint32_t d = dt * 16 + 4 * g4;
          if (d >= value_width) continue;  // padding (a multiple of 8)
          half4_t hv;
#pragma unroll
          for (int e = 0; e < 4; ++e) hv[e] = (half_t)(o[dt][qt][e] * inv);
          *reinterpret_cast<half4_t*>((uint16_t*)out + row + d) = hv;
        }
      }
    }
  } else {
    // fp32 rows go out through LDS: a lane holds 4 columns of one query per
    // d tile, so storing straight from registers writes 64-byte pieces of 16
    // rows per instruction; staged, every instruction writes whole 512-byte
    // row runs.  Each wave stages a 16-query tile (kPassCols columns per
    // pass) in its quarter of the two V stages, which every wave is done
    // reading after this barrier (the K stages may hold the next block's
    // prefetched tile).  Rows of kPassCols fp32, 16-byte chunk c of row r at
    // chunk c ^ (r & 15): a write instruction's 16 rows land on distinct
    // banks.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // Lane indices made opaque here, so the staging addresses are computed
    // now rather than before the key loop (where they would hold registers).
    uint32_t lane_e = lane, r16_e = r16, g4_e = g4;
    asm volatile("" : "+v"(lane_e), "+v"(r16_e), "+v"(g4_e));
    constexpr uint32_t kPassCols = kVTile / 128;  // 16 rows x kPassCols x 4 B = kVTile / 2
    constexpr uint32_t kRowChunks = kPassCols / 4;
    constexpr uint32_t kPasses = (DVC + kPassCols - 1) / kPassCols;
    static_assert(kPassCols % 16 == 0 && kRowChunks <= 32, "whole d tiles per pass, 512-byte rows at most");
    uint8_t* stage = (wave_s < 2 ? lds_v0 : lds_v1) + (wave_s % 2) * (kVTile / 2);
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      const float inv = 1.0f / sum_of_query(l_run[qt]);
#pragma unroll
      for (uint32_t pass = 0; pass < kPasses; ++pass) {
#pragma unroll
        for (uint32_t dt = pass * kPassCols / 16; dt < kDT && dt < (pass + 1) * kPassCols / 16; ++dt) {
          const uint32_t c = (dt - pass * kPassCols / 16) * 4 + g4_e;
          float4_t fv;
#pragma unroll
          for (int e = 0; e < 4; ++e) fv[e] = o[dt][qt][e] * inv;
          *reinterpret_cast<float4_t*>(stage + r16_e * kPassCols * 4 + ((c ^ (r16_e & 15)) << 4)) = fv;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (uint32_t k = 0; k < 16 * kRowChunks / kWave; ++k) {
          const uint32_t v = k * kWave + lane_e, r = v / kRowChunks, c = v % kRowChunks;
          const uint32_t q = wq0 + 16 * qt + r, col = pass * kPassCols + c * 4;
          const float4_t fv = *reinterpret_cast<const float4_t*>(
              stage + r * kPassCols * 4 + ((c ^ (r & 15)) << 4));
          if (q < query_rows && col < value_width)  // a multiple of 8
            *reinterpret_cast<float4_t*>((float*)out + ((uint64_t)stream * query_rows + q) * value_width + col) = fv;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

// One workgroup per pair of query blocks of one stream: 2 i and 2 i + 1
// (non-causal), or n - 1 - i and i (causal: the pair's key steps add up to
// the same count for every workgroup).  When the first block's key block
// count is even, its last step fetches the second block's first K tile and
// its epilogue the second block's Q fragments, so the second block starts
// without a load latency (and without the burst of loads that workgroups
// starting together would issue).  Workgroups are remapped so each XCD
// (round-robin dispatch over 8) runs whole streams, sharing K and V in its L2.
template <int D, int DC, int DV, int DVC, bool Causal, bool OutF16>
__global__ __launch_bounds__(kThreads, 2) void attention_fwd_kernel(
    void* __restrict__ out, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, uint32_t streams, uint32_t query_rows, uint32_t key_rows,
    uint32_t width, uint32_t value_width, float scale_log2, uint32_t q_heads, uint32_t k_heads,
    uint32_t v_heads) {
  constexpr int W = D > DV ? D : DV;
  constexpr uint32_t kQPB = Fast<W>::kQueriesPerBlock;
  const uint32_t qblocks = (query_rows + kQPB - 1) / kQPB;
  const uint32_t per_stream = (qblocks + kBlocksPerGroup - 1) / kBlocksPerGroup;
  const uint32_t total = per_stream * streams;
  uint32_t pid = blockIdx.x;
  if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;  // XCD-contiguous
  const uint32_t stream = pid / per_stream, i = pid % per_stream;
  // Block order within a stream: causal n - 1, 0, n - 2, 1, ... (the heavy
  // block, then its mirror: each pair has the same key steps), otherwise
  // 0, 1, 2, ...; this workgroup runs the pair at positions 2 i, 2 i + 1.
  auto qb_at = [&](uint32_t pos) {
    return Causal ? (pos % 2 == 0 ? qblocks - 1 - pos / 2 : pos / 2) : pos;
  };
  const uint32_t pos0 = i * kBlocksPerGroup;
  const uint32_t reps = qblocks - pos0 < kBlocksPerGroup ? qblocks - pos0 : kBlocksPerGroup;
  half8_t qf[Fast<W>::kQT][DC / 32];
  load_q<W, DC>(qf, query, stream, qb_at(pos0), query_rows, width, q_heads);
  bool loaded = false;  // this block's first K tile and Q fragments were fetched by the last one
  for (uint32_t rep = 0; rep < reps; ++rep) {
    // Every wave is done with the LDS stages before the next block's DMA.
    if (rep > 0) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const uint32_t qb = qb_at(pos0 + rep);
    // A block with an even key block count ends in stage 1, so its last
    // step can fetch the next block's first K tile into stage 0.
    const bool chain = rep + 1 < reps && key_blocks<W, Causal>(qb, query_rows, key_rows) % 2 == 0;
    if (rep > 0 && !loaded) load_q<W, DC>(qf, query, stream, qb, query_rows, width, q_heads);
    attention_block<D, DC, DV, DVC, Causal, OutF16>(out, query, key, value, stream, qb, query_rows,
                                                    key_rows, width, value_width, scale_log2, q_heads,
                                                    k_heads, v_heads, qf, loaded, chain,
                                                    qb_at(pos0 + rep + 1));
    loaded = chain;
  }
}

// MFMA attention for the widths the fast kernel does not take: query/key
// width and value width up to 512, equal or not, multiples of 8
// or not.  256 threads = 4 waves of 16 queries (one 16-query tile each); a
// workgroup runs 64 queries of one stream (the heaviest causal blocks first)
// and shares each block of 32 keys through LDS: the K and V tiles of the
// next block are loaded into registers while the current one computes
// (16-byte loads, or 2-byte loads when a width is not a multiple of 8; zero
// past the key rows and the widths), then stored with the fast kernel's XOR
// swizzles.  S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x32_f16 with
// the fast kernel's lane layouts (a lane holds 4 keys of one query per
// 16-key tile, its probabilities are the output MFMA's operand in place).
// The running maximum is updated every block and the output rescaled, as in
// device/flash_attention_online_f16.cpp:68-143.
namespace wide {
constexpr uint32_t kKeys = 32;
constexpr uint32_t kQueries = 64;  // per workgroup

template <uint32_t DMAX, uint32_t DVMAX, bool Vec8>
__global__ __launch_bounds__(kThreads, DVMAX > 256 ? 1 : 2) void attention_wide_kernel(
    void* __restrict__ out, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, uint32_t query_rows, uint32_t key_rows, uint32_t width,
    uint32_t value_width, float scale_log2, bool causal, bool out_f16, uint32_t q_heads,
    uint32_t k_heads, uint32_t v_heads, uint32_t qblocks) {
  constexpr uint32_t kKRow = DMAX * 2, kVRow = DVMAX * 2;  // LDS row bytes
  constexpr uint32_t kKS = DMAX / 32, kDT = DVMAX / 16;
  constexpr uint32_t kKChunks = DMAX / 8, kVChunks = DVMAX / 8;  // 16-byte chunks a row
  constexpr uint32_t kKPer = kKeys * kKChunks / kThreads, kVPer = kKeys * kVChunks / kThreads;
  static_assert(kKChunks >= 16 && kVChunks >= 16, "swizzles need 16 chunks a row");
  __shared__ __attribute__((aligned(16))) uint8_t lk[kKeys * kKRow];
  __shared__ __attribute__((aligned(16))) uint8_t lv[kKeys * kVRow];

  const uint32_t stream = blockIdx.x / qblocks;
  const uint32_t qb = qblocks - 1 - blockIdx.x % qblocks;
  const uint32_t lane = threadIdx.x % kWave, r16 = lane % 16, g4 = lane / 16;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t q0 = qb * kQueries;
  const uint32_t qi = q0 + wave * 16 + r16;  // this lane's query
  const uint32_t q_pitch = q_heads * width, k_pitch = k_heads * width;
  const uint32_t v_pitch = v_heads * value_width;
  const uint16_t* Q = query + (uint64_t)(stream / q_heads) * query_rows * q_pitch + (stream % q_heads) * width;
  const uint16_t* K = key + (uint64_t)(stream / k_heads) * key_rows * k_pitch + (stream % k_heads) * width;
  const uint16_t* V =
      value + (uint64_t)(stream / v_heads) * key_rows * v_pitch + (stream % v_heads) * value_width;
  const uint32_t nks = (width + 31) / 32, ndt = (value_width + 15) / 16;

  // Elements c .. c + 7 of a row of `limit` elements (zero past it).
  auto load8 = [&](const uint16_t* row, uint32_t c, uint32_t limit) __attribute__((always_inline)) {
    if constexpr (Vec8) {
      return c < limit ? load16(row + c) : u32x4{0, 0, 0, 0};  // limit % 8 == 0
    } else {
      uint32_t w[4];
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t lo = c + 2 * i < limit ? row[c + 2 * i] : 0u;
        const uint32_t hi = c + 2 * i + 1 < limit ? row[c + 2 * i + 1] : 0u;
        w[i] = lo | hi << 16;
      }
      return u32x4{w[0], w[1], w[2], w[3]};
    }
  };

  // Q fragment k step ks: Q[qi][32 ks + 8 (l / 16) .. +7] (rows clamped).
  half8_t qf[kKS];
  {
    const uint32_t q = qi < query_rows ? qi : query_rows - 1;
#pragma unroll
    for (uint32_t ks = 0; ks < kKS; ++ks)
      qf[ks] = __builtin_bit_cast(half8_t, load8(Q + (uint64_t)q * q_pitch, 32 * ks + 8 * g4, width));
  }

  uint32_t key_end = key_rows;
  if (causal) {
    const uint32_t last_q = q0 + kQueries < query_rows ? q0 + kQueries : query_rows;
    key_end = last_q < key_rows ? last_q : key_rows;
  }
  const uint32_t nblocks = (key_end + kKeys - 1) / kKeys;

  // Tile chunk i of this thread: row (i * 256 + t) / chunks, chunk % chunks.
  u32x4 rk[kKPer], rv[kVPer];
  auto load_tiles = [&](uint32_t kb) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t i = 0; i < kKPer; ++i) {
      const uint32_t c = i * kThreads + threadIdx.x, row = c / kKChunks, ch = c % kKChunks;
      rk[i] = kb + row < key_rows ? load8(K + (uint64_t)(kb + row) * k_pitch, 8 * ch, width)
                                  : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (uint32_t i = 0; i < kVPer; ++i) {
      const uint32_t c = i * kThreads + threadIdx.x, row = c / kVChunks, ch = c % kVChunks;
      rv[i] = kb + row < key_rows ? load8(V + (uint64_t)(kb + row) * v_pitch, 8 * ch, value_width)
                                  : u32x4{0, 0, 0, 0};
    }
  };
  auto store_tiles = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t i = 0; i < kKPer; ++i) {
      const uint32_t c = i * kThreads + threadIdx.x, row = c / kKChunks, ch = c % kKChunks;
      *reinterpret_cast<u32x4*>(lk + row * kKRow + ((ch ^ (row & 15u)) << 4)) = rk[i];
    }
#pragma unroll
    for (uint32_t i = 0; i < kVPer; ++i) {
      const uint32_t c = i * kThreads + threadIdx.x, row = c / kVChunks, ch = c % kVChunks;
      *reinterpret_cast<u32x4*>(lv + row * kVRow + ((ch ^ ((row & 7u) << 1)) << 4)) = rv[i];
    }
  };
  const uint32_t kbase = r16 * kKRow + ((g4 ^ (r16 & 15u)) << 4);
  uint32_t vbase;
  {
    const uint32_t row = 4 * g4 + r16 / 4, c1 = (r16 % 4) / 2;
    vbase = row * kVRow + ((c1 ^ ((row & 7u) << 1)) << 4) + 8 * (r16 % 2);
  }

  float4_t o[kDT];
#pragma unroll
  for (uint32_t dt = 0; dt < kDT; ++dt) o[dt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY, l_run = 0.0f;

  load_tiles(0);
  for (uint32_t b = 0; b < nblocks; ++b) {
    const uint32_t kb = b * kKeys;
    __syncthreads();  // every wave is done with the previous tiles
    store_tiles();
    __syncthreads();
    if (b + 1 < nblocks) load_tiles(kb + kKeys);
    // Scores: s[kt][e] = key kb + 16 kt + 4 (l / 16) + e of query qi.
    float4_t s[2];
#pragma unroll
    for (uint32_t kt = 0; kt < 2; ++kt) {
      s[kt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (uint32_t ks = 0; ks < kKS; ++ks) {
        if (ks < nks) {
          const half8_t kf = __builtin_bit_cast(
              half8_t, *reinterpret_cast<const u32x4*>(lk + (kbase ^ (ks << 6)) + 16 * kt * kKRow));
          s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], s[kt], 0, 0, 0);
        }
      }
    }
    // Online softmax in log2 units; masked keys are -inf.  A query whose
    // keys in this block are all masked keeps its reference point (every
    // query has key 0 in block 0).
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t kt = 0; kt < 2; ++kt)
#pragma unroll
      for (uint32_t e = 0; e < 4; ++e) {
        const uint32_t k = kb + 16 * kt + 4 * g4 + e;
        const bool ok = k < key_rows && (!causal || k <= qi);
        s[kt][e] = ok ? s[kt][e] * scale_log2 : -INFINITY;
        mx = fmaxf(mx, s[kt][e]);
      }
    mx = max_of_query(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    half8_t pp;
    float sum = 0.0f;
#pragma unroll
    for (uint32_t e = 0; e < 8; ++e) {
      const float p = __builtin_amdgcn_exp2f(s[e / 4][e % 4] - m_use);
      pp[e] = (half_t)p;
      sum += (float)pp[e];
    }
    l_run = l_run * alpha + sum;
    // Output: o[dt][e] = O^T[d = 16 dt + 4 (l / 16) + e][qi].
#pragma unroll
    for (uint32_t dt = 0; dt < kDT; ++dt) {
      if (dt < ndt) {
        const uint8_t* p = lv + (vbase ^ (dt << 5));
        const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)p);
        const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)(p + 16 * kVRow));
        const half8_t vf = __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pp, o[dt] * alpha, 0, 0, 0);
      }
    }
  }
  const float inv = 1.0f / sum_of_query(l_run);
  if (qi >= query_rows) return;
  const uint64_t row = ((uint64_t)stream * query_rows + qi) * value_width;
#pragma unroll
  for (uint32_t dt = 0; dt < kDT; ++dt) {
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) {
      const uint32_t d = dt * 16 + 4 * g4 + e;
      if (d >= value_width) continue;
      const float r = o[dt][e] * inv;
      if (out_f16)
        ((uint16_t*)out)[row + d] = __builtin_bit_cast(uint16_t, (half_t)r);
      else
        ((float*)out)[row + d] = r;
    }
  }
}

template <uint32_t DMAX, uint32_t DVMAX>
int launch(hipStream_t stream, const AttentionArgs& a, float scale_log2, bool vec8) {
  const uint32_t qblocks = (a.query_rows + kQueries - 1) / kQueries;
  const uint64_t blocks = (uint64_t)qblocks * a.streams;
  if (blocks > 0x7fffffffu) return IPUS_ERROR_INVALID_ARGUMENT;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((uint32_t)blocks), dim3(kThreads), 0, stream, a.out,
                       (const uint16_t*)a.query, (const uint16_t*)a.key, (const uint16_t*)a.value,
                       a.query_rows, a.key_rows, a.width, a.value_width, scale_log2, a.causal,
                       a.output_f16, a.heads[0], a.heads[1], a.heads[2], qblocks);
  };
  if (vec8) go(attention_wide_kernel<DMAX, DVMAX, true>);
  else go(attention_wide_kernel<DMAX, DVMAX, false>);
  return hip_status(hipGetLastError());
}
}  // namespace wide

// One 64-lane block per (stream, query row): the fallback for query/key
// widths above 512 (any query/key width, value width up to 512).
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

template <int D, int DC, int DV, int DVC, bool Causal, bool OutF16>
int launch_fast(hipStream_t stream, const AttentionArgs& a, float scale_log2) {
  constexpr uint32_t kQPB = Fast<(D > DV ? D : DV)>::kQueriesPerBlock;
  const uint32_t qblocks = (a.query_rows + kQPB - 1) / kQPB;
  const uint64_t blocks = (uint64_t)((qblocks + kBlocksPerGroup - 1) / kBlocksPerGroup) * a.streams;
  if (blocks > 0x7fffffffu) return IPUS_ERROR_INVALID_ARGUMENT;
  hipLaunchKernelGGL((attention_fwd_kernel<D, DC, DV, DVC, Causal, OutF16>), dim3((uint32_t)blocks),
                     dim3(kThreads), 0, stream, a.out, (const uint16_t*)a.query,
                     (const uint16_t*)a.key, (const uint16_t*)a.value, a.streams, a.query_rows,
                     a.key_rows, a.width, a.value_width, scale_log2, a.heads[0], a.heads[1],
                     a.heads[2]);
  return hip_status(hipGetLastError());
}

// Tile widths D / DV (LDS rows, DMA) and computed columns DC / DVC (score
// k steps / output tiles) of the query-key and value widths.
template <int D, int DC, int DV = D, int DVC = DC>
int dispatch_fast(hipStream_t stream, const AttentionArgs& a, float scale_log2) {
  if (a.causal)
    return a.output_f16 ? launch_fast<D, DC, DV, DVC, true, true>(stream, a, scale_log2)
                        : launch_fast<D, DC, DV, DVC, true, false>(stream, a, scale_log2);
  return a.output_f16 ? launch_fast<D, DC, DV, DVC, false, true>(stream, a, scale_log2)
                      : launch_fast<D, DC, DV, DVC, false, false>(stream, a, scale_log2);
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
  // Every kernel holds a row pitch (heads x width elements) in 32 bits.
  if ((uint64_t)a.heads[0] * a.width > 0xffffffffull || (uint64_t)a.heads[1] * a.width > 0xffffffffull ||
      (uint64_t)a.heads[2] * a.value_width > 0xffffffffull)
    return IPUS_ERROR_INVALID_ARGUMENT;
  // The fast kernel addresses one stream's K or V through a buffer
  // descriptor with a 31-bit byte range; the offsets of the last block's
  // rows (up to 63 past the end) and of padding chunks stay below 2^32.
  const uint64_t k_pitch = (uint64_t)a.heads[1] * a.width * 2, v_pitch = (uint64_t)a.heads[2] * a.value_width * 2;
  const uint64_t kv_pitch = k_pitch > v_pitch ? k_pitch : v_pitch;
  const bool fits = ((uint64_t)a.key_rows + kMaxKeysPerBlock) * kv_pitch <= 0x7fff0000ull;
  // Equal widths that are multiples of 8 up to 256 run in 64-, 128- or
  // 256-wide tiles (zero padding), computing 32, 64, 96, 128, 192 or 256
  // columns; other widths take the MFMA kernel below, or the
  // one-row-per-block kernel past its limits.
  if (aligned && fits && a.width == a.value_width && a.width % 8 == 0 && a.width <= 256) {
    if (a.width > 192) return dispatch_fast<256, 256>(stream, a, scale_log2);
    if (a.width > 128) return dispatch_fast<256, 192>(stream, a, scale_log2);
    if (a.width > 96) return dispatch_fast<128, 128>(stream, a, scale_log2);
    if (a.width > 64) return dispatch_fast<128, 96>(stream, a, scale_log2);
    if (a.width > 32) return dispatch_fast<64, 64>(stream, a, scale_log2);
    return dispatch_fast<64, 32>(stream, a, scale_log2);
  }
  // Unequal widths, multiples of 8, whose tile widths (64, 128 or 256 each)
  // are one of these pairs: the same kernel with separate K and V tiles.
  if (aligned && fits && a.width % 8 == 0 && a.value_width % 8 == 0 && a.width <= 256 &&
      a.value_width <= 256) {
    auto tile = [](uint32_t w) { return w <= 64 ? 64u : w <= 128 ? 128u : 256u; };
    const uint32_t tq = tile(a.width), tv = tile(a.value_width);
    if (tq == 128 && tv == 64) return dispatch_fast<128, 128, 64, 64>(stream, a, scale_log2);
    if (tq == 64 && tv == 128) return dispatch_fast<64, 64, 128, 128>(stream, a, scale_log2);
    if (tq == 256 && tv == 128) return dispatch_fast<256, 256, 128, 128>(stream, a, scale_log2);
    if (tq == 128 && tv == 256) return dispatch_fast<128, 128, 256, 256>(stream, a, scale_log2);
  }
  // Query/key and value widths up to 512: the MFMA kernel for other widths,
  // in the smallest of its tile classes that holds them.
  if (a.width <= 512 && a.value_width <= 512) {
    const bool vec8 = aligned && a.width % 8 == 0 && a.value_width % 8 == 0;
    if (a.width <= 128 && a.value_width <= 128) return wide::launch<128, 128>(stream, a, scale_log2, vec8);
    if (a.width <= 256 && a.value_width <= 256) return wide::launch<256, 256>(stream, a, scale_log2, vec8);
    if (a.width <= 256) return wide::launch<256, 512>(stream, a, scale_log2, vec8);
    return wide::launch<512, 512>(stream, a, scale_log2, vec8);
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
