// Fused online-softmax attention on gfx950 MFMA:
//   O = softmax(scale * Q K^T [+ causal mask]) V
// Q, K, V fp16 [streams, rows, width]; fp32 scores, running max and sum;
// fp32 output by default (the reference's device attention output precision,
// crates/ipu-codegen/src/mid.rs:2064-2067) or fp16.  Semantics:
// device/flash_attention_online_f16.cpp:68-143 (online softmax, exact) and
// crates/ipu-tests/src/diagnostic.rs:711-780 (key j allowed iff j <= i when
// causal, 741-745; scale default 1/sqrt(width), 733-736).
//
// Fast kernel (width == value width in {64, 128}):
//   * 256 threads = 4 waves; a wave owns 64 queries (two 32-query tiles), a
//     block 256 queries of one stream; keys stream through LDS in blocks of 64
//     with two stages (next block's loads in flight during the math);
//   * scores are computed transposed, S^T = K Q^T, with
//     v_mfma_f32_32x32x16_f16 (K rows from LDS as the first operand, Q
//     fragments resident in registers as the second), so each lane holds 16
//     keys of ONE query: the row max needs one cross-lane exchange (lane ^ 32)
//     and the running sum none until the end;
//   * the output is accumulated transposed too, O^T += V^T P^T: the fp16
//     probabilities are the second MFMA operand straight from the score
//     registers (no shuffle), because V^T is stored in LDS with its keys
//     permuted to match the score accumulator layout; the rescale by
//     exp(m_old - m_new) is lane-local;
//   * causal: key blocks past the block's last query are never loaded, a wave
//     skips blocks past its own last query, and blocks are issued heaviest
//     first.
#include "../../include/ipus.h"
#include "device_common.h"
#include "kernels.h"

namespace ipus {
namespace {

constexpr int kThreads = 256;
constexpr int kQueriesPerBlock = 256;
constexpr int kKeysPerBlock = 64;
constexpr float kLog2e = 1.4426950408889634f;

inline int hip_status(hipError_t e) { return e == hipSuccess ? 0 : IPUS_ERROR_HIP_BASE - (int)e; }

// K tile: [64 keys][D] fp16, rows of D*2 bytes, 16-byte chunks XOR (key & 7).
template <int D>
__device__ __forceinline__ uint32_t k_off(uint32_t key, uint32_t chunk) {
  return key * (D * 2) + ((chunk ^ (key & 7u)) << 4);
}
// V^T tile: [D][64 key slots] fp16, 128-byte rows, chunks XOR ((d ^ d>>3) & 7).
__device__ __forceinline__ uint32_t vt_off(uint32_t d, uint32_t chunk) {
  return d * 128u + ((chunk ^ ((d ^ (d >> 3)) & 7u)) << 4);
}

// Key slot inside a 32-key group: key = 8a + 4g + b is stored at slot
// (a/2)*16 + g*8 + (a%2)*4 + b, so that PV MFMA h of the group reads, in lane
// group g, the 8 keys {8(2h)+4g+b, 8(2h+1)+4g+b} that score accumulator
// elements 8h..8h+7 of that lane hold.

template <int D>
struct Tiles {
  static constexpr uint32_t kBytes = kKeysPerBlock * D * 2;  // per operand
};

// Threads 128..255 load K (D/8 * 64 / 128 vectors each), threads 0..127 load
// V as 8x8 blocks (one block per thread for D = 128, half for D = 64).
template <int D>
struct KvRegs {
  u32x4 v[8];
};

template <int D>
__device__ __forceinline__ void load_kv(const uint16_t* __restrict__ K,
                                        const uint16_t* __restrict__ V, uint32_t key0,
                                        uint32_t key_rows, KvRegs<D>& r) {
  const uint32_t t = threadIdx.x;
  constexpr uint32_t chunks = D / 8;  // 16-byte chunks per row
  if (t >= 128) {
    const uint32_t u = t - 128;
    // 64 rows x chunks vectors over 128 threads.
    constexpr uint32_t per = 64 * chunks / 128;
#pragma unroll
    for (uint32_t i = 0; i < per; ++i) {
      const uint32_t idx = u + 128 * i;
      uint32_t key = key0 + idx / chunks;
      key = key < key_rows ? key : key_rows - 1;
      r.v[i] = load16(K + (uint64_t)key * D + (idx % chunks) * 8);
    }
  } else {
    // 8x8 blocks: key group kg (8 groups), d chunk dc (chunks).  D=128: 128
    // blocks, one per thread; D=64: 64 blocks on threads 0..63.
    if (t < 8 * chunks) {
      const uint32_t dc = t % chunks, kg = t / chunks;
#pragma unroll
      for (uint32_t j = 0; j < 8; ++j) {
        uint32_t key = key0 + kg * 8 + j;
        key = key < key_rows ? key : key_rows - 1;
        r.v[j] = load16(V + (uint64_t)key * D + dc * 8);
      }
    }
  }
}

template <int D>
__device__ __forceinline__ void store_kv(uint8_t* lds_k, uint8_t* lds_vt, const KvRegs<D>& r) {
  const uint32_t t = threadIdx.x;
  constexpr uint32_t chunks = D / 8;
  if (t >= 128) {
    const uint32_t u = t - 128;
    constexpr uint32_t per = 64 * chunks / 128;
#pragma unroll
    for (uint32_t i = 0; i < per; ++i) {
      const uint32_t idx = u + 128 * i;
      *reinterpret_cast<u32x4*>(lds_k + k_off<D>(idx / chunks, idx % chunks)) = r.v[i];
    }
  } else if (t < 8 * chunks) {
    const uint32_t dc = t % chunks, kg = t / chunks;
    u32x4 w[8];
    transpose8x8_u16(r.v, w);
    // w[i] = keys kg*8 .. kg*8+7 of d = dc*8 + i.
    const uint32_t group32 = kg / 4;  // which 32-key group
    const uint32_t a = kg % 4;        // keys 8a .. 8a+7 of the group
    const uint32_t h = a / 2, half = a % 2;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const uint32_t d = dc * 8 + i;
      // keys 8a+0..3 -> g = 0, keys 8a+4..7 -> g = 1; each a 4-slot run at
      // byte offset half*8 inside chunk group32*4 + h*2 + g.
      uint8_t* base0 = lds_vt + vt_off(d, group32 * 4 + h * 2 + 0) + half * 8;
      uint8_t* base1 = lds_vt + vt_off(d, group32 * 4 + h * 2 + 1) + half * 8;
      *reinterpret_cast<u32x2*>(base0) = u32x2{w[i][0], w[i][1]};
      *reinterpret_cast<u32x2*>(base1) = u32x2{w[i][2], w[i][3]};
    }
  }
}

template <int D, bool Causal, bool OutF16>
__global__ __launch_bounds__(kThreads, 1) void attention_fwd_kernel(
    void* __restrict__ out, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, uint32_t streams, uint32_t query_rows, uint32_t key_rows,
    float scale_log2) {
  constexpr uint32_t kDT = D / 32;  // output d tiles
  constexpr uint32_t kKS = D / 16;  // k steps of the score MFMA
  constexpr uint32_t kBytes = Tiles<D>::kBytes;
  __shared__ __attribute__((aligned(16))) uint8_t smem[4 * kBytes];

  const uint32_t qblocks = (query_rows + kQueriesPerBlock - 1) / kQueriesPerBlock;
  const uint32_t stream = blockIdx.x % streams;
  const uint32_t qb = Causal ? qblocks - 1 - blockIdx.x / streams : blockIdx.x / streams;
  const uint32_t q0 = qb * kQueriesPerBlock;
  const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const uint32_t wq0 = q0 + wave * 64;  // first query of this wave

  const uint16_t* Q = query + (uint64_t)stream * query_rows * D;
  const uint16_t* K = key + (uint64_t)stream * key_rows * D;
  const uint16_t* V = value + (uint64_t)stream * key_rows * D;

  // Q fragments (second MFMA operand): lane holds Q[q][16 ks + 8 (lane/32) ..+7].
  half8_t qf[2][kKS];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    uint32_t q = wq0 + qt * 32 + lane % 32;
    q = q < query_rows ? q : query_rows - 1;
#pragma unroll
    for (uint32_t ks = 0; ks < kKS; ++ks)
      qf[qt][ks] = __builtin_bit_cast(half8_t, load16(Q + (uint64_t)q * D + ks * 16 + (lane / 32) * 8));
  }

  float16_t o[2][kDT];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (uint32_t dt = 0; dt < kDT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[qt][dt][e] = 0.0f;
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.0f, 0.0f};

  uint32_t key_end = key_rows;
  if (Causal) {
    const uint32_t last_q = (q0 + kQueriesPerBlock < query_rows ? q0 + kQueriesPerBlock : query_rows);
    key_end = last_q < key_rows ? last_q : key_rows;  // keys <= last query
  }
  const uint32_t nblocks = (key_end + kKeysPerBlock - 1) / kKeysPerBlock;
  const uint32_t wave_last_q = wq0 + 63;

  KvRegs<D> regs;
  load_kv<D>(K, V, 0, key_rows, regs);
  store_kv<D>((smem + 0 + (0) * 2 * kBytes), (smem + kBytes + (0) * 2 * kBytes), regs);
  __syncthreads();

  for (uint32_t kbi = 0; kbi < nblocks; ++kbi) {
    const uint32_t cur = kbi & 1;
    const uint32_t kb = kbi * kKeysPerBlock;
    const bool more = kbi + 1 < nblocks;
    if (more) load_kv<D>(K, V, kb + kKeysPerBlock, key_rows, regs);

    const bool active = !Causal || kb <= wave_last_q;
    if (active) {
      const uint8_t* lk = (smem + 0 + (cur) * 2 * kBytes);
      const uint8_t* lv = (smem + kBytes + (cur) * 2 * kBytes);
      const bool need_mask = (Causal && kb + kKeysPerBlock - 1 > wq0) || kb + kKeysPerBlock > key_rows;
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        // Scores S^T for 64 keys (two 32-key tiles) x 32 queries.
        float16_t s[2];
#pragma unroll
        for (int st = 0; st < 2; ++st) {
#pragma unroll
          for (int e = 0; e < 16; ++e) s[st][e] = 0.0f;
#pragma unroll
          for (uint32_t ks = 0; ks < kKS; ++ks) {
            const half8_t kf = __builtin_bit_cast(
                half8_t, *reinterpret_cast<const u32x4*>(
                             lk + k_off<D>(st * 32 + lane % 32, ks * 2 + lane / 32)));
            s[st] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[qt][ks], s[st], 0, 0, 0);
          }
        }
        // s[st][r] is key kb + 32 st + 8 (r/4) + 4 (lane/32) + r%4 of query
        // wq0 + 32 qt + lane % 32.
        const uint32_t qi = wq0 + qt * 32 + lane % 32;
        float mx = -INFINITY;
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float v = s[st][r] * scale_log2;
            if (need_mask) {
              const uint32_t kj = kb + 32 * st + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
              if ((Causal && kj > qi) || kj >= key_rows) v = -INFINITY;
            }
            s[st][r] = v;
            mx = fmaxf(mx, v);
          }
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float m_new = fmaxf(m_run[qt], mx);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = exp2f(m_run[qt] - m_use);
        m_run[qt] = m_new;
        float psum = 0.0f;
        half8_t pf[2][2];
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float p = exp2f(s[st][8 * h + e] - m_use);
              psum += p;
              pf[st][h][e] = (half_t)p;
            }
        l_run[qt] = l_run[qt] * alpha + psum;
#pragma unroll
        for (uint32_t dt = 0; dt < kDT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[qt][dt][e] *= alpha;
        // O^T += V^T P^T over the 64 keys: 4 MFMAs (st, h) per d tile.
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (uint32_t dt = 0; dt < kDT; ++dt) {
              const half8_t vf = __builtin_bit_cast(
                  half8_t, *reinterpret_cast<const u32x4*>(
                               lv + vt_off(dt * 32 + lane % 32, st * 4 + h * 2 + lane / 32)));
              o[qt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[st][h], o[qt][dt], 0, 0, 0);
            }
      }
    }
    if (more) store_kv<D>((smem + 0 + (cur ^ 1) * 2 * kBytes), (smem + kBytes + (cur ^ 1) * 2 * kBytes), regs);
    __syncthreads();
  }

  // o[qt][dt][r] = O^T[d = 32 dt + 8 (r/4) + 4 (lane/32) + r%4][q].
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float l_total = l_run[qt] + __shfl_xor(l_run[qt], 32, kWave);
    const float inv = 1.0f / l_total;
    const uint32_t q = wq0 + qt * 32 + lane % 32;
    if (q >= query_rows) continue;
    const uint64_t row = ((uint64_t)stream * query_rows + q) * D;
#pragma unroll
    for (uint32_t dt = 0; dt < kDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t d = dt * 32 + 8 * g + 4 * (lane / 32);
        if constexpr (OutF16) {
          half4_t hv;
#pragma unroll
          for (int e = 0; e < 4; ++e) hv[e] = (half_t)(o[qt][dt][4 * g + e] * inv);
          *reinterpret_cast<half4_t*>((uint16_t*)out + row + d) = hv;
        } else {
          float4_t fv;
#pragma unroll
          for (int e = 0; e < 4; ++e) fv[e] = o[qt][dt][4 * g + e] * inv;
          *reinterpret_cast<float4_t*>((float*)out + row + d) = fv;
        }
      }
  }
}

// General attention: one 64-lane block per (stream, query row); any widths.
// Online softmax over keys one at a time (dot products by wave reduction).
constexpr uint32_t kGeneralMaxValuePerLane = 8;  // value width <= 512

__global__ __launch_bounds__(64) void attention_general_kernel(
    void* __restrict__ out, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, uint32_t query_rows, uint32_t key_rows, uint32_t width,
    uint32_t value_width, float scale_log2, bool causal, bool out_f16) {
  const uint64_t flat = blockIdx.x;
  const uint32_t stream = (uint32_t)(flat / query_rows);
  const uint32_t row = (uint32_t)(flat % query_rows);
  const uint32_t lane = threadIdx.x;
  const uint16_t* q = query + flat * width;
  const uint16_t* K = key + (uint64_t)stream * key_rows * width;
  const uint16_t* V = value + (uint64_t)stream * key_rows * value_width;
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
             (float)__builtin_bit_cast(half_t, K[(uint64_t)j * width + d]);
    dot = wave_sum(dot) * scale_log2;
    const float m_new = fmaxf(m, dot);
    const float alpha = exp2f(m - m_new);
    const float p = exp2f(dot - m_new);
    l = l * alpha + p;
#pragma unroll
    for (uint32_t i = 0; i < kGeneralMaxValuePerLane; ++i) {
      const uint32_t c = lane + 64 * i;
      const float v = c < value_width ? (float)__builtin_bit_cast(half_t, V[(uint64_t)j * value_width + c]) : 0.0f;
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
  const uint64_t blocks = (uint64_t)qblocks * a.streams;
  if (blocks > 0x7fffffffu) return IPUS_ERROR_INVALID_ARGUMENT;
  hipLaunchKernelGGL((attention_fwd_kernel<D, Causal, OutF16>), dim3((uint32_t)blocks),
                     dim3(kThreads), 0, stream, a.out, (const uint16_t*)a.query,
                     (const uint16_t*)a.key, (const uint16_t*)a.value, a.streams, a.query_rows,
                     a.key_rows, scale_log2);
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
  if (aligned && a.width == a.value_width && (a.width == 128 || a.width == 64)) {
    return a.width == 128 ? dispatch_fast<128>(stream, a, scale_log2)
                          : dispatch_fast<64>(stream, a, scale_log2);
  }
  if (a.value_width > 64 * kGeneralMaxValuePerLane) return IPUS_ERROR_UNAVAILABLE;
  const uint64_t blocks = (uint64_t)a.streams * a.query_rows;
  if (blocks > 0x7fffffffu) return IPUS_ERROR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(attention_general_kernel, dim3((uint32_t)blocks), dim3(64), 0, stream, a.out,
                     (const uint16_t*)a.query, (const uint16_t*)a.key, (const uint16_t*)a.value,
                     a.query_rows, a.key_rows, a.width, a.value_width, scale_log2, a.causal,
                     a.output_f16);
  return hip_status(hipGetLastError());
}

}  // namespace ipus
