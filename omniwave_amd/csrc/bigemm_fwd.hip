// Fused BiGEMM forward for gfx950 (CDNA4): RMSNorm row statistics, weight packing, the tile
// kernel and the C-ABI launchers.
//
// Math per tile (omniweave/ops/reference.py:147-171): for the 16 routed tokens of a token
// group and the d routed channels of a channel group,
//     delta = A_o . (SiLU(A_u . T . B_u) * (A_v . T . B_v)) . B_o      scaled per column by gamma
// evaluated with the cheapest association, P = A.T first and Z.B_o before A_o.  With the
// block's RMSNorm fused, T = diag(r) X diag(w) (r = per-token rsqrt scale, w = norm weight),
// so P^T = diag(w) X^T (A diag(r))^T: r scales the A operand of each token group and w is
// folded into the packed B_u / B_v rows.  SiLU's exponent base is folded into the weights too:
// B_u' = -log2(e) B_u, B_v' = -ln(2) B_v give U' = -log2(e) U, V' = -ln(2) V and
//     SiLU(U) V = U V / (1 + e^-U) = U' V' / (1 + 2^U').
//
// MFMA layouts (64 lanes; l16 = lane % 16, h = lane / 16, l32 = lane % 32, hh = lane / 32):
//   16x16 accumulator        lane holds D[4h + i][l16], i = 0..3
//   16x16x16 A / B operand   lane holds A[l16][4h + j] / B[4h + j][l16], j = 0..3
//   32x32 accumulator        lane holds D[8(i/4) + 4hh + i%4][l32], i = 0..15
//   32x32x16 A / B operand   lane holds 8 K-slots j = 0..7 of row / column l32 for K half hh
// Only the pairing of A slot (hh, j) with B slot (hh, j) is fixed by the hardware, so each
// operand may use any K order as long as both sides agree.  All products are computed
// transposed (tokens on the MFMA N axis) so every result feeds the next contraction from
// registers:
//     P^T  = X^T . (A diag r)^T  16x16x16 per token group (K = 16 tokens), X^T from LDS;
//            two groups' results are merged into one 32-token B operand by a lane exchange
//     U'^T = B_u'^T . P_u^T      32x32x16 (K = channels, N = 32 tokens), weights from LDS
//     Z^T  = U'V' / (1 + 2^U')   registers; a 32-row accumulator block is two 16-deep
//                                K steps of the next product
//     W^T  = B_o^T . Z^T         32x32x16 (K = expanded dim)
//     delta = A_o . W            16x16x16 per token group, W transposed through LDS
// Weights are pre-packed (ow_pack_weights) so each MFMA operand is one 16-byte LDS read per
// lane, and each chunk of weights is copied global -> LDS directly (global_load_lds).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_common.h"

namespace ow {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kG = 16;        // spatial tile (tokens per group)
constexpr int kWaves = 4;     // waves per workgroup
constexpr int kThreads = 256;
constexpr int kTokFragElems = 256;             // 16x16x16 operand: 64 lanes x 4
constexpr int kHeadElems = 3 * kTokFragElems;  // A_u^T, A_v^T, A_o at the head of `packed`
constexpr int kFragElems = 512;                // 32x32x16 operand: 64 lanes x 8
constexpr float kNegLog2e = -1.4426950408889634f;
constexpr float kNegLn2 = -0.6931471805599453f;

struct BF16 {
  static __device__ __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  static __device__ __forceinline__ float to_f32(uint16_t u) {
    return __uint_as_float(static_cast<uint32_t>(u) << 16);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
  // a.lo^2 + a.hi^2 + acc in fp32
  static __device__ __forceinline__ float dot2sq(uint32_t a, float acc) {
    const bf16x2 v = __builtin_bit_cast(bf16x2, a);
    return __builtin_amdgcn_fdot2_f32_bf16(v, v, acc, false);
  }
  static __device__ __forceinline__ f32x16 mma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                     __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
  }
};

struct F16 {
  static __device__ __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
  static __device__ __forceinline__ float to_f32(uint16_t u) {
    return static_cast<float>(__builtin_bit_cast(_Float16, u));
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  static __device__ __forceinline__ float dot2sq(uint32_t a, float acc) {
    const f16x2 v = __builtin_bit_cast(f16x2, a);
    return __builtin_amdgcn_fdot2(v, v, acc, false);
  }
  static __device__ __forceinline__ f32x16 mma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
};

template <class Ty>
__device__ __forceinline__ float round_to(float f) {
  return Ty::to_f32(Ty::from_f32(f));
}

// RMSNorm row scale with the reference's dtype sequence (omniweave/models/block.py:83-84):
// var (fp32) -> x.dtype, + eps in x.dtype, rsqrt in x.dtype.
template <class Ty>
__device__ __forceinline__ float rms_scale(float mean_sq, float eps) {
  const float v = round_to<Ty>(round_to<Ty>(mean_sq) + eps);
  return round_to<Ty>(rsqrtf(v));
}

// SiLU(U) V from the folded accumulators U' = -log2(e) U, V' = -ln(2) V.
__device__ __forceinline__ float silu_gate(float up, float vp) {
  return up * vp * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(up));
}

// Separates MFMA results from VALU reads of them by 32 wait states.  Used where the read
// follows the MFMA across a basic-block boundary (loop exit), or where many accumulator
// registers are read at once: the hardware does not interlock an MFMA's result against a
// later VALU read, and a read a few instructions after a 16x16x16 MFMA returns the old value
// of its last accumulator register.  The scheduling barriers keep the compiler from moving
// MFMAs or reads across the padding.
__device__ __forceinline__ void mfma_drain() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Makes this wave's LDS writes visible to its other lanes before they read them.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint16_t lo16(uint32_t v) { return static_cast<uint16_t>(v & 0xffffu); }
__device__ __forceinline__ uint16_t hi16(uint32_t v) { return static_cast<uint16_t>(v >> 16); }

// ---------------------------------------------------------------------------------------
// RMSNorm row scales: scale[row] = rsqrt(mean(x[row]^2) + eps) in the reference's dtype
// sequence, one fp32 value per token.  Vector path: VPRW = C/8 16-byte vectors per row,
// LPR = min(64, VPRW) lanes per row, 8 rows per wave.

struct RmsArgs {
  const uint16_t* x;
  float* scale;
  int64_t rows;
  int32_t channels;
  float eps;
};

template <class Ty, int VPRW>
__global__ void __launch_bounds__(kThreads) rms_rows_kernel(RmsArgs a) {
  constexpr int LPR = VPRW < 64 ? VPRW : 64;
  constexpr int RPI = 64 / LPR;   // rows per wave instruction
  constexpr int NR = 8 / RPI;     // rows per lane
  constexpr int VPL = VPRW / LPR; // vectors per lane per row
  static_assert(RPI <= 8, "at least 8 lanes per row");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % LPR;
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * 8;
  u32x4 v[NR][VPL];
#pragma unroll
  for (int rr = 0; rr < NR; ++rr) {
    const int64_t row = base + rr * RPI + lane / LPR;
#pragma unroll
    for (int q = 0; q < VPL; ++q) {
      v[rr][q] = u32x4{0u, 0u, 0u, 0u};
      if (row < a.rows)
        v[rr][q] = *reinterpret_cast<const u32x4*>(a.x + row * a.channels + (sub + q * LPR) * 8);
    }
  }
#pragma unroll
  for (int rr = 0; rr < NR; ++rr) {
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < VPL; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = Ty::dot2sq(v[rr][q][e], acc);
#pragma unroll
    for (int m = LPR >> 1; m > 0; m >>= 1) acc += __shfl_xor(acc, m);
    const int64_t row = base + rr * RPI + lane / LPR;
    if (sub == 0 && row < a.rows) a.scale[row] = rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps);
  }
}

// Any C: one wave per row, element loads.
template <class Ty>
__global__ void __launch_bounds__(kThreads) rms_rows_generic_kernel(RmsArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  if (row >= a.rows) return;
  float acc = 0.0f;
  for (int c = lane; c < a.channels; c += 64) {
    const float v = Ty::to_f32(a.x[row * a.channels + c]);
    acc = fmaf(v, v, acc);
  }
  for (int m = 32; m > 0; m >>= 1) acc += __shfl_xor(acc, m);
  if (lane == 0) a.scale[row] = rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps);
}

// ---------------------------------------------------------------------------------------
// Tile kernel.

struct FwdArgs {
  const uint16_t* x;
  uint16_t* out;
  const float* row_scale;  // [batch * n_tok] RMSNorm scale per token, NULL without OW_FUSE_NORM
  const float* gamma;      // [C]
  const uint16_t* packed;
  const int32_t* tok;
  const int32_t* chan;
  int32_t batch, n_tok, channels, q_s, q_c;
  int32_t n_chunks;  // ceil(batch * q_s / token groups per workgroup)
  int32_t residual;  // write x + delta instead of delta
  int32_t gather;    // element-wise channel gather/scatter (rotated or padded channel groups)
};

// Maps the hardware workgroup id to a logical id so that the q_c workgroups of one row chunk
// run on the same XCD (workgroups are dispatched round-robin over the 8 XCDs): their gathers
// and scatters touch the same cache lines of x and out, which then meet in one L2.
__device__ __forceinline__ int xcd_remap(int bid, int nwg) {
  const int xcd = bid & 7, slot = bid >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + slot;
}

// Direct global -> LDS copy of one 1 KB operand fragment by one wave (16 bytes per lane).
__device__ __forceinline__ void copy_frag_to_lds(const uint16_t* src, uint16_t* dst, int lane) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + lane * 8),
                                   (__attribute__((address_space(3))) void*)(dst), 16, 0, 0);
}

__device__ __forceinline__ void wait_lds_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// One workgroup: 4 waves x TPW token groups (TPW/2 pairs of 16 tokens per wave) x one channel
// group q_c.
template <class Ty, int D, int RD, int TPW, int OCC>
__global__ void __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads), amdgpu_waves_per_eu(OCC)))
bigemm_fwd_kernel(FwdArgs a) {
  constexpr int NP = TPW / 2;      // token-group pairs per wave (32-token MFMA N blocks)
  constexpr int R = kWaves * TPW;  // token groups per workgroup
  constexpr int ROWS = R * kG;
  constexpr int LDX = D + 8;       // padded LDS row stride (elements): conflict-free column reads
  constexpr int KS = D / 16;       // 16-deep K steps over the channel tile (= 16-channel blocks)
  constexpr int MB = D / 32;       // 32-channel output blocks of W^T
  constexpr int NCH = RD / 32;     // 32-row chunks of the expanded dimension
  constexpr int FR_U = KS;         // B_u'^T fragments per chunk (B_v'^T the same)
  constexpr int FR_O = 2 * MB;     // B_o^T fragments per chunk (MB blocks x 2 K steps)
  constexpr int FR_CH = 2 * FR_U + FR_O;
  constexpr int CH_ELEMS = FR_CH * kFragElems;
  static_assert(TPW % 2 == 0, "token groups come in pairs");
  static_assert(CH_ELEMS <= ROWS * LDX, "a weight chunk must fit in the x-tile region");

  // LDS regions.  xs: the x tile until the token side has read it; then the odd weight
  // chunks; after the chunk loop, each wave's W^T tile (its own 32 rows) and then delta.
  // wb: the even weight chunks.
  __shared__ __attribute__((aligned(16))) uint16_t xs[ROWS * LDX];
  __shared__ __attribute__((aligned(16))) uint16_t wb[CH_ELEMS];
  __shared__ int32_t rowid[ROWS];  // b * n_tok + token, -1 for pad rows
  __shared__ float rsc[ROWS];      // RMSNorm scale of each row (1 without norm)
  __shared__ float gm[D];
  __shared__ int32_t chx[D];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, h = lane >> 4;
  const int tau = (lane >> 4) & 1;  // which token group of a pair this lane's MFMA column is in

  const int bid = xcd_remap(blockIdx.x, a.n_chunks * a.q_c);
  const int qc = bid % a.q_c, chunk = bid / a.q_c;

  const uint16_t* wsrc = a.packed + kHeadElems + static_cast<size_t>(qc) * NCH * CH_ELEMS;
  auto chunk_buf = [&](int ec) -> uint16_t* { return (ec & 1) ? xs : wb; };
  auto issue_chunk = [&](int ec) {
    const uint16_t* src = wsrc + static_cast<size_t>(ec) * CH_ELEMS;
    uint16_t* dst = chunk_buf(ec);
    for (int f = wave; f < FR_CH; f += kWaves) copy_frag_to_lds(src + f * kFragElems, dst + f * kFragElems, lane);
  };
  issue_chunk(0);

  for (int r = tid; r < ROWS; r += kThreads) {
    const int64_t tg = static_cast<int64_t>(chunk) * R + r / kG;
    int32_t id = -1;
    if (tg < static_cast<int64_t>(a.batch) * a.q_s) {
      const int32_t b = static_cast<int32_t>(tg / a.q_s);
      const int32_t s = static_cast<int32_t>(tg - static_cast<int64_t>(b) * a.q_s);
      const int32_t t = a.tok[s * kG + (r % kG)];
      if (t >= 0 && t < a.n_tok) id = b * a.n_tok + t;
    }
    rowid[r] = id;
    rsc[r] = (id >= 0 && a.row_scale) ? a.row_scale[id] : 1.0f;
  }
  for (int k = tid; k < D; k += kThreads) {
    const int c = a.chan[qc * D + k];
    const bool ok = c >= 0 && c < a.channels;
    chx[k] = ok ? c : -1;
    gm[k] = ok ? a.gamma[c] : 0.0f;
  }
  __syncthreads();

  // x tile [ROWS x D] into LDS (pad rows / columns read as zero).
  if (!a.gather) {
    constexpr int VPR = D / 8;
    constexpr int NV = ROWS * VPR / kThreads;
    u32x4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + i * kThreads;
      const int64_t id = rowid[idx / VPR];
      v[i] = u32x4{0u, 0u, 0u, 0u};
      if (id >= 0) v[i] = *reinterpret_cast<const u32x4*>(a.x + id * a.channels + qc * D + (idx % VPR) * 8);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + i * kThreads;
      *reinterpret_cast<u32x4*>(&xs[(idx / VPR) * LDX + (idx % VPR) * 8]) = v[i];
    }
  } else {
    for (int i = tid; i < ROWS * D; i += kThreads) {
      const int r = i / D, k = i % D;
      const int64_t id = rowid[r];
      const int c = chx[k];
      xs[r * LDX + k] = (id >= 0 && c >= 0) ? a.x[id * a.channels + c] : static_cast<uint16_t>(0);
    }
  }

  const u32x2 fAu = reinterpret_cast<const u32x2*>(a.packed)[lane];
  const u32x2 fAv = reinterpret_cast<const u32x2*>(a.packed + kTokFragElems)[lane];
  const u32x2 fAo = reinterpret_cast<const u32x2*>(a.packed + 2 * kTokFragElems)[lane];
  __syncthreads();

  // Token side.  For a pair (groups 0, 1) and 16-channel block kb, S_g = 16x16 result of group
  // g (lane holds channels kb*16 + 4h + i of token l16).  The 32x32x16 B operand wants, in lane
  // L = 32hh + 16tau + t, channels kb*16 + 8hh + j (j = 0..7) of token t of group tau: slots 0-3
  // live in lane 32hh + t and slots 4-7 in lane 32hh + 16 + t of S_tau.  A lane of group tau
  // owns one half and receives the other from lane L ^ 16, which sends its S_(1-tau).
  const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  u32x4 Pu[NP][KS], Pv[NP][KS];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    u32x2 bu[2], bv[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int row0 = (wave * TPW + 2 * p + g) * kG;
      bu[g] = fAu;
      bv[g] = fAv;
      if (a.row_scale) {  // lane holds A[l16][4h + j]: scale by r of row 4h + j
        const float r0 = rsc[row0 + 4 * h + 0], r1 = rsc[row0 + 4 * h + 1];
        const float r2 = rsc[row0 + 4 * h + 2], r3 = rsc[row0 + 4 * h + 3];
        bu[g] = u32x2{Ty::pack2(Ty::to_f32(lo16(fAu[0])) * r0, Ty::to_f32(hi16(fAu[0])) * r1),
                      Ty::pack2(Ty::to_f32(lo16(fAu[1])) * r2, Ty::to_f32(hi16(fAu[1])) * r3)};
        bv[g] = u32x2{Ty::pack2(Ty::to_f32(lo16(fAv[0])) * r0, Ty::to_f32(hi16(fAv[0])) * r1),
                      Ty::pack2(Ty::to_f32(lo16(fAv[1])) * r2, Ty::to_f32(hi16(fAv[1])) * r3)};
      }
    }
#pragma unroll
    for (int kb = 0; kb < KS; ++kb) {
      u32x2 su[2], sv[2];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int row0 = (wave * TPW + 2 * p + g) * kG;
        const int k = kb * 16 + l16;
        const uint32_t e0 = xs[(row0 + 4 * h + 0) * LDX + k];
        const uint32_t e1 = xs[(row0 + 4 * h + 1) * LDX + k];
        const uint32_t e2 = xs[(row0 + 4 * h + 2) * LDX + k];
        const uint32_t e3 = xs[(row0 + 4 * h + 3) * LDX + k];
        const u32x2 av = {e0 | (e1 << 16), e2 | (e3 << 16)};
        const f32x4 pu = Ty::mma16(av, bu[g], zero4);
        const f32x4 pv = Ty::mma16(av, bv[g], zero4);
        su[g] = u32x2{Ty::pack2(pu[0], pu[1]), Ty::pack2(pu[2], pu[3])};
        sv[g] = u32x2{Ty::pack2(pv[0], pv[1]), Ty::pack2(pv[2], pv[3])};
      }
      const u32x2 send_u = tau ? su[0] : su[1], own_u = tau ? su[1] : su[0];
      const u32x2 send_v = tau ? sv[0] : sv[1], own_v = tau ? sv[1] : sv[0];
      const u32x2 recv_u = {static_cast<uint32_t>(__shfl_xor(static_cast<int>(send_u[0]), 16)),
                            static_cast<uint32_t>(__shfl_xor(static_cast<int>(send_u[1]), 16))};
      const u32x2 recv_v = {static_cast<uint32_t>(__shfl_xor(static_cast<int>(send_v[0]), 16)),
                            static_cast<uint32_t>(__shfl_xor(static_cast<int>(send_v[1]), 16))};
      Pu[p][kb] = tau ? u32x4{recv_u[0], recv_u[1], own_u[0], own_u[1]} : u32x4{own_u[0], own_u[1], recv_u[0], recv_u[1]};
      Pv[p][kb] = tau ? u32x4{recv_v[0], recv_v[1], own_v[0], own_v[1]} : u32x4{own_v[0], own_v[1], recv_v[0], recv_v[1]};
    }
  }

  // Channel side, streamed over 32-row chunks of the expanded dimension (double-buffered).
  f32x16 W[NP][MB];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) W[p][mb][i] = 0.0f;

  for (int ec = 0; ec < NCH; ++ec) {
    wait_lds_dma();
    // Chunk ec has landed; every wave is done with chunk ec - 1 (and, at ec = 0, with the x
    // tile), so the buffer of chunk ec + 1 is free.
    __syncthreads();
    if (ec + 1 < NCH) issue_chunk(ec + 1);
    const uint16_t* cw = chunk_buf(ec);
    f32x16 U[NP], V[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int i = 0; i < 16; ++i) U[p][i] = V[p][i] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const u32x4 fu = reinterpret_cast<const u32x4*>(cw + ks * kFragElems)[lane];
      const u32x4 fv = reinterpret_cast<const u32x4*>(cw + (FR_U + ks) * kFragElems)[lane];
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        U[p] = Ty::mma32(fu, Pu[p][ks], U[p]);
        V[p] = Ty::mma32(fv, Pv[p][ks], V[p]);
      }
    }
    // Z^T chunk: accumulator registers 8s..8s+7 are K step s (16 rows) of the next product.
    u32x4 Z[NP][2];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          Z[p][s][q] = Ty::pack2(silu_gate(U[p][8 * s + 2 * q], V[p][8 * s + 2 * q]),
                                 silu_gate(U[p][8 * s + 2 * q + 1], V[p][8 * s + 2 * q + 1]));
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4 fo = reinterpret_cast<const u32x4*>(cw + (2 * FR_U + 2 * mb + s) * kFragElems)[lane];
#pragma unroll
        for (int p = 0; p < NP; ++p) W[p][mb] = Ty::mma32(fo, Z[p][s], W[p][mb]);
      }
  }

  // Output side: each wave stages W^T of a pair into its own 32 rows of xs (transposed to
  // [token][channel]), computes delta = A_o . W per group with LayerScale, and writes the
  // rounded delta over the same rows.  W^T lane layout: c = 32mb + 8(i/4) + 4hh + i%4,
  // token column lane % 32.  No branch separates an MFMA from the reads of its result.
  mfma_drain();
  __syncthreads();  // every wave is done with the last weight chunk
  const int hh = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    uint16_t* st = xs + (wave * TPW + 2 * p) * kG * LDX;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const u32x2 v = {Ty::pack2(W[p][mb][4 * gi + 0], W[p][mb][4 * gi + 1]),
                         Ty::pack2(W[p][mb][4 * gi + 2], W[p][mb][4 * gi + 3])};
        *reinterpret_cast<u32x2*>(st + l32 * LDX + mb * 32 + 8 * gi + 4 * hh) = v;
      }
    wave_lds_sync();
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      uint16_t* sg = st + (16 * g) * LDX;
      f32x4 dl[KS];
#pragma unroll
      for (int nb = 0; nb < KS; ++nb) {
        const int k = nb * 16 + l16;
        const uint32_t e0 = sg[(4 * h + 0) * LDX + k];
        const uint32_t e1 = sg[(4 * h + 1) * LDX + k];
        const uint32_t e2 = sg[(4 * h + 2) * LDX + k];
        const uint32_t e3 = sg[(4 * h + 3) * LDX + k];
        const u32x2 bw = {e0 | (e1 << 16), e2 | (e3 << 16)};
        dl[nb] = Ty::mma16(fAo, bw, zero4);
      }
      mfma_drain();  // also orders this group's W reads before the delta writes below
#pragma unroll
      for (int nb = 0; nb < KS; ++nb) {
        const int k = nb * 16 + l16;
        const float gmv = gm[k];
#pragma unroll
        for (int i = 0; i < 4; ++i) sg[(4 * h + i) * LDX + k] = Ty::from_f32(dl[nb][i] * gmv);
      }
    }
    wave_lds_sync();
  }
  __syncthreads();

  // out = round(x + delta) (x re-read from global memory, normally an L2 hit) or delta.
  if (!a.gather) {
    constexpr int VPR = D / 8;
    for (int i = tid; i < ROWS * VPR; i += kThreads) {
      const int r = i / VPR, v = i % VPR;
      const int64_t id = rowid[r];
      if (id < 0) continue;
      u32x4 dv = *reinterpret_cast<const u32x4*>(&xs[r * LDX + v * 8]);
      const int64_t off = id * a.channels + qc * D + v * 8;
      if (a.residual) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(a.x + off);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          dv[q] = Ty::pack2(Ty::to_f32(lo16(xv[q])) + Ty::to_f32(lo16(dv[q])),
                            Ty::to_f32(hi16(xv[q])) + Ty::to_f32(hi16(dv[q])));
      }
      *reinterpret_cast<u32x4*>(a.out + off) = dv;
    }
  } else {
    for (int i = tid; i < ROWS * D; i += kThreads) {
      const int r = i / D, k = i % D;
      const int64_t id = rowid[r];
      const int c = chx[k];
      if (id < 0 || c < 0) continue;
      const int64_t off = id * a.channels + c;
      const uint16_t dv = xs[r * LDX + k];
      a.out[off] = a.residual ? Ty::from_f32(Ty::to_f32(a.x[off]) + Ty::to_f32(dv)) : dv;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Weight packing.

struct PackArgs {
  const void* a_u;
  const void* a_v;
  const void* a_o;
  const void* b_u;
  const void* b_v;
  const void* b_o;
  const float* norm_w;  // folded into B_u / B_v rows (NULL: weight 1)
  const int32_t* chan;  // channel table [q_c * d] (routes norm_w to tile rows)
  void* packed;
  int32_t wdtype, q_c, d, rd, channels;
  int64_t total;
};

__device__ __forceinline__ float load_f32(const void* p, int64_t i, int dtype) {
  if (dtype == OW_DTYPE_F32) return static_cast<const float*>(p)[i];
  const uint16_t u = static_cast<const uint16_t*>(p)[i];
  return dtype == OW_DTYPE_BF16 ? BF16::to_f32(u) : F16::to_f32(u);
}

// Packed order: [A_u^T | A_v^T | A_o] 16x16x16 operands, then per (q, chunk ec): KS B_u'^T
// fragments, KS B_v'^T fragments, 2*MB B_o^T fragments (32x32x16 A operands, 64 lanes x 8).
//   B_u'^T / B_v'^T, K step ks: lane l slot j -> row e = 32ec + l32, channel 16ks + 8hh + j
//                               (the channel order the token-side lane exchange produces)
//   B_o^T (mb, s):              lane l slot j -> row c = 32mb + l32, expanded index
//                               32ec + 16s + 8(j/4) + 4hh + j%4 (accumulator rows of U^T)
template <class Ty>
__global__ void __launch_bounds__(256) pack_kernel(PackArgs p) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= p.total) return;
  float val;
  if (idx < kHeadElems) {
    // Token-side 16x16x16 operands: lane l slot j -> A[l16][4h + j].
    const int frag = static_cast<int>(idx / kTokFragElems);
    const int e = static_cast<int>(idx % kTokFragElems);
    const int lane = e / 4, j = e % 4;
    const int src = (lane & 15) * kG + 4 * (lane >> 4) + j;
    val = load_f32(frag == 0 ? p.a_u : frag == 1 ? p.a_v : p.a_o, src, p.wdtype);
  } else {
    const int ks_n = p.d / 16, mb_n = p.d / 32, nch = p.rd / 32;
    const int64_t ch_elems = static_cast<int64_t>(2 * ks_n + 2 * mb_n) * kFragElems;
    int64_t rem = idx - kHeadElems;
    const int q = static_cast<int>(rem / (nch * ch_elems));
    rem -= static_cast<int64_t>(q) * nch * ch_elems;
    const int ec = static_cast<int>(rem / ch_elems);
    rem -= static_cast<int64_t>(ec) * ch_elems;
    const int fr = static_cast<int>(rem / kFragElems);
    const int e = static_cast<int>(rem % kFragElems);
    const int lane = e / 8, j = e % 8;
    const int l32 = lane & 31, hh = lane >> 5;
    if (fr < 2 * ks_n) {
      const bool is_u = fr < ks_n;
      const int ks = fr % ks_n;
      const int col = 32 * ec + l32;
      const int c = 16 * ks + 8 * hh + j;
      const int64_t src = (static_cast<int64_t>(q) * p.d + c) * p.rd + col;
      float w = 1.0f;
      if (p.norm_w) {
        const int gc = p.chan[q * p.d + c];
        w = (gc >= 0 && gc < p.channels) ? p.norm_w[gc] : 0.0f;
      }
      val = load_f32(is_u ? p.b_u : p.b_v, src, p.wdtype) * w * (is_u ? kNegLog2e : kNegLn2);
    } else {
      const int f = fr - 2 * ks_n;
      const int mb = f / 2, s = f % 2;
      const int c = 32 * mb + l32;
      const int ee = 32 * ec + 16 * s + 8 * (j / 4) + 4 * hh + (j % 4);
      const int64_t src = (static_cast<int64_t>(q) * p.rd + ee) * p.d + c;
      val = load_f32(p.b_o, src, p.wdtype);
    }
  }
  static_cast<uint16_t*>(p.packed)[idx] = Ty::from_f32(val);
}

int64_t packed_elems(int32_t q_c, int32_t d, int32_t rd) {
  const int64_t per_chunk = static_cast<int64_t>(2 * (d / 16) + 2 * (d / 32)) * kFragElems;
  return kHeadElems + static_cast<int64_t>(q_c) * (rd / 32) * per_chunk;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return OW_OK;
  return fail(OW_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

template <class Ty>
int launch_rms(const RmsArgs& a, hipStream_t s) {
  const int vprw = a.channels % 8 == 0 ? a.channels / 8 : 0;
  const unsigned blocks8 = static_cast<unsigned>((a.rows + kWaves * 8 - 1) / (kWaves * 8));
  switch (vprw) {
    case 8: hipLaunchKernelGGL((rms_rows_kernel<Ty, 8>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 16: hipLaunchKernelGGL((rms_rows_kernel<Ty, 16>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 32: hipLaunchKernelGGL((rms_rows_kernel<Ty, 32>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 64: hipLaunchKernelGGL((rms_rows_kernel<Ty, 64>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 128: hipLaunchKernelGGL((rms_rows_kernel<Ty, 128>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    case 256: hipLaunchKernelGGL((rms_rows_kernel<Ty, 256>), dim3(blocks8), dim3(kThreads), 0, s, a); break;
    default: {
      const unsigned blocks = static_cast<unsigned>((a.rows + kWaves - 1) / kWaves);
      hipLaunchKernelGGL(rms_rows_generic_kernel<Ty>, dim3(blocks), dim3(kThreads), 0, s, a);
    }
  }
  return hip_status(hipGetLastError(), "rms_rows_kernel launch");
}

// Token groups per wave (TPW) and workgroups per CU (OCC) for the two channel tiles.
#ifndef OW_TPW_D128
#define OW_TPW_D128 2
#endif
#ifndef OW_OCC_D128
#define OW_OCC_D128 2
#endif
#ifndef OW_TPW_D64
#define OW_TPW_D64 2
#endif
#ifndef OW_OCC_D64
#define OW_OCC_D64 3
#endif

// d = 128: 4 token groups per wave (two 32-token MFMA blocks share each weight fragment read
// from LDS), one workgroup per CU.  d = 64: the same tiling fits two workgroups per CU.
template <class Ty, int D, int RD>
int launch_fwd(const FwdArgs& a, hipStream_t stream) {
  constexpr int TPW = D == 64 ? OW_TPW_D64 : OW_TPW_D128;
  constexpr int OCC = D == 64 ? OW_OCC_D64 : OW_OCC_D128;
  constexpr int R = kWaves * TPW;
  FwdArgs args = a;
  const int64_t groups = static_cast<int64_t>(a.batch) * a.q_s;
  const int64_t chunks = (groups + R - 1) / R;
  const int64_t nwg = chunks * a.q_c;
  if (nwg == 0) return OW_OK;
  if (nwg > 0x7fffffff) return fail(OW_ERR_UNSUPPORTED, "grid too large (%lld workgroups)", (long long)nwg);
  args.n_chunks = static_cast<int32_t>(chunks);
  hipLaunchKernelGGL((bigemm_fwd_kernel<Ty, D, RD, TPW, OCC>), dim3(static_cast<unsigned>(nwg)), dim3(kThreads),
                     0, stream, args);
  return hip_status(hipGetLastError(), "bigemm_fwd_kernel launch");
}

template <class Ty>
int dispatch_fwd(const FwdArgs& a, int d, int rd, hipStream_t s) {
  if (d == 64 && rd == 128) return launch_fwd<Ty, 64, 128>(a, s);
  if (d == 64 && rd == 256) return launch_fwd<Ty, 64, 256>(a, s);
  if (d == 128 && rd == 128) return launch_fwd<Ty, 128, 128>(a, s);
  if (d == 128 && rd == 256) return launch_fwd<Ty, 128, 256>(a, s);
  return fail(OW_ERR_UNSUPPORTED, "unsupported channel tile d=%d / expanded dim rd=%d; expected d in {64,128}, rd in {128,256}", d, rd);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace ow

extern "C" {

size_t ow_packed_weight_bytes(int32_t q_c, int32_t d, int32_t rd, int32_t compute_dtype) {
  if (q_c < 1 || d < 32 || rd < 32 || d % 32 || rd % 32) return 0;
  const size_t elem = compute_dtype == OW_DTYPE_F32 ? 4 : 2;
  return static_cast<size_t>(ow::packed_elems(q_c, d, rd)) * elem;
}

size_t ow_fwd_workspace_bytes(const OwPlan* plan, int32_t batch, int32_t flags) {
  if (!plan || batch < 0 || !(flags & OW_FUSE_NORM)) return 0;
  return static_cast<size_t>(batch) * static_cast<size_t>(plan->height) * static_cast<size_t>(plan->width) *
         sizeof(float);
}

int ow_pack_weights(const void* a_u, const void* a_v, const void* a_o, const void* b_u, const void* b_v,
                    const void* b_o, int32_t weight_dtype, const float* norm_weight, const int32_t* channel_index,
                    int32_t channels, int32_t g, int32_t q_c, int32_t d, int32_t rd, int32_t compute_dtype,
                    void* packed, void* stream) {
  OW_CHECK_ARG(a_u && a_v && a_o && b_u && b_v && b_o && packed, "weight or output pointer is NULL");
  OW_CHECK_ARG(!norm_weight || channel_index, "norm_weight needs channel_index");
  OW_CHECK_ARG(channels >= 1, "channels must be >= 1 (got %d)", channels);
  OW_CHECK_ARG(weight_dtype >= OW_DTYPE_F32 && weight_dtype <= OW_DTYPE_F16, "unknown weight dtype %d", weight_dtype);
  OW_CHECK_SUPPORTED(g == ow::kG, "unsupported spatial tile g=%d; expected 16", g);
  OW_CHECK_ARG(q_c >= 1, "q_c must be >= 1 (got %d)", q_c);
  OW_CHECK_SUPPORTED((d == 64 || d == 128) && (rd == 128 || rd == 256),
                     "unsupported channel tile d=%d / expanded dim rd=%d", d, rd);
  OW_CHECK_SUPPORTED(compute_dtype == OW_DTYPE_BF16 || compute_dtype == OW_DTYPE_F16,
                     "unsupported compute dtype %d", compute_dtype);
  ow::PackArgs p{a_u, a_v, a_o, b_u, b_v, b_o, norm_weight, channel_index, packed,
                 weight_dtype, q_c, d, rd, channels, ow::packed_elems(q_c, d, rd)};
  const unsigned blocks = static_cast<unsigned>((p.total + 255) / 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (compute_dtype == OW_DTYPE_BF16)
    hipLaunchKernelGGL(ow::pack_kernel<ow::BF16>, dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(ow::pack_kernel<ow::F16>, dim3(blocks), dim3(256), 0, s, p);
  if (int rc = ow::hip_status(hipGetLastError(), "pack_kernel launch")) return rc;
  ow::clear_error();
  return OW_OK;
}

int ow_rms_scale(const void* x, float* scale, int64_t rows, int32_t channels, float eps, int32_t dtype,
                 void* stream) {
  OW_CHECK_ARG(rows >= 0 && channels >= 1, "bad shape rows=%lld channels=%d", (long long)rows, channels);
  if (rows == 0) {
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(x && scale, "tensor pointer is NULL");
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16, "unsupported dtype %d", dtype);
  ow::RmsArgs r{static_cast<const uint16_t*>(x), scale, rows, channels, eps};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!ow::aligned16(x)) {  // element path
    const unsigned blocks = static_cast<unsigned>((rows + ow::kWaves - 1) / ow::kWaves);
    if (dtype == OW_DTYPE_BF16)
      hipLaunchKernelGGL(ow::rms_rows_generic_kernel<ow::BF16>, dim3(blocks), dim3(ow::kThreads), 0, s, r);
    else
      hipLaunchKernelGGL(ow::rms_rows_generic_kernel<ow::F16>, dim3(blocks), dim3(ow::kThreads), 0, s, r);
    if (int rc = ow::hip_status(hipGetLastError(), "rms_rows_generic_kernel launch")) return rc;
  } else {
    const int rc = dtype == OW_DTYPE_BF16 ? ow::launch_rms<ow::BF16>(r, s) : ow::launch_rms<ow::F16>(r, s);
    if (rc) return rc;
  }
  ow::clear_error();
  return OW_OK;
}

int ow_bigemm_fwd(const void* x, void* out, float eps, const float* gamma, const void* packed,
                  size_t packed_bytes, const int32_t* token_index, const int32_t* channel_index,
                  const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype, int32_t flags, void* workspace,
                  size_t workspace_bytes, void* stream) {
  int32_t q_s = 0, q_c = 0;
  if (int rc = ow_plan_dims(plan, &q_s, &q_c)) return rc;
  OW_CHECK_ARG(batch >= 0, "batch must be >= 0 (got %d)", batch);
  OW_CHECK_ARG(gamma && packed && token_index && channel_index, "tensor pointer is NULL");
  OW_CHECK_ARG((flags & ~(OW_FUSE_NORM | OW_FUSE_RESIDUAL)) == 0, "unknown flags 0x%x", flags);
  OW_CHECK_SUPPORTED(plan->spatial_tile == ow::kG, "unsupported spatial tile g=%d; expected 16", plan->spatial_tile);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16,
                     "unsupported dtype %d; expected bf16 or f16", dtype);
  const int32_t n = plan->height * plan->width, c = plan->channels, d = plan->channel_tile;
  const size_t want = ow_packed_weight_bytes(q_c, d, rd, dtype);
  OW_CHECK_ARG(want != 0 && packed_bytes == want,
               "packed weights hold %zu bytes; q_c=%d d=%d rd=%d needs %zu", packed_bytes, q_c, d, rd, want);
  OW_CHECK_ARG(ow::aligned16(packed), "packed weights must be 16-byte aligned");
  if (batch == 0) {  // empty tensors may carry NULL data pointers; nothing to launch
    ow::clear_error();
    return OW_OK;
  }
  OW_CHECK_ARG(x && out, "tensor pointer is NULL");
  OW_CHECK_ARG(x != out, "out must not alias x");
  OW_CHECK_ARG(static_cast<int64_t>(batch) * n * c < (int64_t(1) << 40), "tensor too large");
  OW_CHECK_ARG(static_cast<int64_t>(batch) * n < (int64_t(1) << 31), "batch * H * W must be < 2^31");
  const size_t need_ws = ow_fwd_workspace_bytes(plan, batch, flags);
  OW_CHECK_ARG(workspace_bytes >= need_ws && (need_ws == 0 || workspace),
               "workspace holds %zu bytes; %zu needed", workspace_bytes, need_ws);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* scale = nullptr;
  if (flags & OW_FUSE_NORM) {
    scale = static_cast<float*>(workspace);
    if (int rc = ow_rms_scale(x, scale, static_cast<int64_t>(batch) * n, c, eps, dtype, stream)) return rc;
  }
  ow::FwdArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.out = static_cast<uint16_t*>(out);
  a.row_scale = scale;
  a.gamma = gamma;
  a.packed = static_cast<const uint16_t*>(packed);
  a.tok = token_index;
  a.chan = channel_index;
  a.batch = batch;
  a.n_tok = n;
  a.channels = c;
  a.q_s = q_s;
  a.q_c = q_c;
  a.residual = (flags & OW_FUSE_RESIDUAL) ? 1 : 0;
  const bool contig = (c % d == 0) && (plan->radix_level == 0 || q_c <= 1);
  const bool vec_ok = (c % 8 == 0) && ow::aligned16(x) && ow::aligned16(out);
  a.gather = !(contig && vec_ok);
  const int rc = dtype == OW_DTYPE_BF16 ? ow::dispatch_fwd<ow::BF16>(a, d, rd, s)
                                        : ow::dispatch_fwd<ow::F16>(a, d, rd, s);
  if (rc == OW_OK) ow::clear_error();
  return rc;
}

}  // extern "C"
