// Fused BiGEMM forward for gfx950 (CDNA4): weight packing + the tile kernel + C-ABI launchers.
//
// Math per tile (omniweave/ops/reference.py:147-171): for the 16 routed tokens of a token
// group and the d routed channels of a channel group,
//     delta = A_o . (SiLU(A_u . T . B_u) * (A_v . T . B_v)) . B_o      scaled per column by gamma
// evaluated with the cheapest association, P = A.T first and Z.B_o before A_o.
//
// MFMA layout facts used throughout (64 lanes, l16 = lane % 16, h = lane / 16):
//   16x16 accumulator      lane holds D[4h + i][l16], i = 0..3
//   16x16x16 A operand     lane holds A[l16][4h + j], j = 0..3
//   16x16x16 B operand     lane holds B[4h + j][l16]
//   16x16x32 A / B operand lane holds 8 K-slots j = 0..7 of row/column l16; only the pairing
//                          of A slot (h, j) with B slot (h, j) matters, so K index
//                          kk(h, j) = 16*(j/4) + 4h + (j%4) is used for both.
// With that K map, two stacked 16x16 accumulator blocks (rows 0-15 and 16-31) are, after
// rounding to bf16/fp16, exactly a 16x16x32 B operand whose K runs over those 32 rows.  All
// products are therefore computed transposed (tokens on the MFMA N axis) so every
// accumulator feeds the next contraction from registers:
//     P^T = T^T . A^T          (16x16x16, K = tokens)           T^T from LDS
//     U^T = B_u^T . P_u^T      (16x16x32, K = channels)         weights from LDS
//     Z^T = SiLU(U^T) * V^T    (registers)
//     W^T = B_o^T . Z^T        (16x16x32, K = expanded dim)
//     delta = A_o . W          (16x16x16, K = tokens)           W transposed through LDS
// Weights are pre-packed (ow_pack_weights) so each MFMA operand is one 16-byte LDS read per
// lane.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ow_common.h"

namespace ow {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kG = 16;        // spatial tile (tokens per group)
constexpr int kWaves = 4;     // waves per workgroup
constexpr int kThreads = 256;
constexpr int kTokFragElems = 256;           // 16x16x16 operand: 64 lanes x 4
constexpr int kHeadElems = 3 * kTokFragElems;  // A_u^T, A_v^T, A_o at the head of `packed`
constexpr int kFragElems = 512;              // 16x16x32 operand: 64 lanes x 8

struct BF16 {
  static __device__ __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  static __device__ __forceinline__ float to_f32(uint16_t u) {
    return __uint_as_float(static_cast<uint32_t>(u) << 16);
  }
  static __device__ __forceinline__ f32x4 mma32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
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
  static __device__ __forceinline__ f32x4 mma32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
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

template <class Ty>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return static_cast<uint32_t>(Ty::from_f32(lo)) | (static_cast<uint32_t>(Ty::from_f32(hi)) << 16);
}

// RMSNorm row scale with the reference's dtype sequence (omniweave/models/block.py:83-84):
// var (fp32) -> x.dtype, + eps in x.dtype, rsqrt in x.dtype.
template <class Ty>
__device__ __forceinline__ float rms_scale(float mean_sq, float eps) {
  const float v = round_to<Ty>(round_to<Ty>(mean_sq) + eps);
  return round_to<Ty>(rsqrtf(v));
}

__device__ __forceinline__ float silu_gate(float u, float v) {
  return u * v * __builtin_amdgcn_rcpf(1.0f + __expf(-u));
}

// Makes this wave's LDS writes visible to its other lanes before they read them.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct FwdArgs {
  const uint16_t* x;
  uint16_t* out;
  const float* norm_w;
  const float* gamma;
  const uint16_t* packed;
  const int32_t* tok;
  const int32_t* chan;
  int32_t batch, n_tok, channels, q_s, q_c;
  int32_t n_chunks;     // ceil(batch * q_s / token groups per workgroup)
  int32_t flags;
  float eps;
  int32_t chan_contig;  // channel_index[q*D + k] == q*D + k for every q, k (no pad columns)
  int32_t vec_ok;       // C % 8 == 0 and x/out 16-byte aligned
};

// Maps the hardware workgroup id to a logical id so that the q_c workgroups of one row chunk
// (which all read the same full rows for the RMSNorm statistics) run on the same XCD and
// share its L2.  Workgroups are dispatched round-robin over the 8 XCDs.
__device__ __forceinline__ int xcd_remap(int bid, int nwg) {
  const int xcd = bid & 7, slot = bid >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + slot;
}

// One workgroup: TPW token groups per wave (4 waves) x one channel group q_c.
template <class Ty, int D, int RD, int TPW>
__global__ void __launch_bounds__(kThreads) bigemm_fwd_kernel(FwdArgs a) {
  constexpr int R = kWaves * TPW;  // token groups per workgroup
  constexpr int ROWS = R * kG;
  constexpr int LDX = D + 8;       // padded LDS row stride (elements): conflict-free column reads
  constexpr int KS = D / 32;       // 32-wide K steps over the channel tile
  constexpr int MB = D / 16;       // 16-channel blocks
  constexpr int NCH = RD / 32;     // 32-wide chunks of the expanded dimension
  constexpr int FR_U = 2 * KS;     // B_u^T fragments per chunk (2 e-blocks x KS)
  constexpr int FR_CH = 2 * FR_U + MB;
  constexpr int CH_ELEMS = FR_CH * kFragElems;
  constexpr int CH_VEC = CH_ELEMS / 8;
  constexpr int PF = (CH_VEC + kThreads - 1) / kThreads;

  __shared__ __attribute__((aligned(16))) uint16_t xs[ROWS * LDX];
  __shared__ __attribute__((aligned(16))) uint16_t wst[kWaves][kG * LDX];
  __shared__ __attribute__((aligned(16))) uint16_t wb[CH_ELEMS];
  __shared__ float rrow[ROWS];
  __shared__ int64_t rowoff[ROWS];
  __shared__ float wn[D];
  __shared__ float gm[D];
  __shared__ int32_t chx[D];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, h = lane >> 4;
  const bool fuse_norm = (a.flags & OW_FUSE_NORM) != 0;
  const bool fuse_res = (a.flags & OW_FUSE_RESIDUAL) != 0;

  const int bid = xcd_remap(blockIdx.x, a.n_chunks * a.q_c);
  const int qc = bid % a.q_c, chunk = bid / a.q_c;

  for (int r = tid; r < ROWS; r += kThreads) {
    const int64_t tg = static_cast<int64_t>(chunk) * R + r / kG;
    int64_t off = -1;
    if (tg < static_cast<int64_t>(a.batch) * a.q_s) {
      const int64_t b = tg / a.q_s;
      const int s = static_cast<int>(tg - b * a.q_s);
      const int t = a.tok[s * kG + (r % kG)];
      if (t >= 0 && t < a.n_tok) off = (b * a.n_tok + t) * a.channels;
    }
    rowoff[r] = off;
  }
  for (int k = tid; k < D; k += kThreads) {
    const int c = a.chan[qc * D + k];
    const bool ok = c >= 0 && c < a.channels;
    chx[k] = ok ? c : -1;
    wn[k] = (ok && fuse_norm) ? a.norm_w[c] : 1.0f;
    gm[k] = ok ? a.gamma[c] : 0.0f;
  }
  __syncthreads();

  // RMSNorm statistics over the full C-row of each of this wave's rows.
  {
    const int rbase = wave * TPW * kG;
    if (!fuse_norm) {
      for (int r = lane; r < TPW * kG; r += 64) rrow[rbase + r] = 1.0f;
    } else if (a.vec_ok) {
      const int lpr = a.channels >= 512 ? 64 : a.channels >= 256 ? 32 : a.channels >= 128 ? 16
                    : a.channels >= 64 ? 8 : 4;
      const int rpi = 64 / lpr;
      const int sub = lane & (lpr - 1);
      for (int r0 = 0; r0 < TPW * kG; r0 += rpi) {
        const int r = rbase + r0 + lane / lpr;
        const int64_t off = rowoff[r];
        float acc = 0.0f;
        if (off >= 0) {
          for (int c = sub * 8; c < a.channels; c += lpr * 8) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(a.x + off + c);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float lo = Ty::to_f32(static_cast<uint16_t>(v[q] & 0xffffu));
              const float hi = Ty::to_f32(static_cast<uint16_t>(v[q] >> 16));
              acc = fmaf(lo, lo, acc);
              acc = fmaf(hi, hi, acc);
            }
          }
        }
        for (int m = lpr >> 1; m > 0; m >>= 1) acc += __shfl_xor(acc, m);
        if (sub == 0) rrow[r] = rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps);
      }
    } else {
      for (int r = rbase; r < rbase + TPW * kG; ++r) {
        const int64_t off = rowoff[r];
        float acc = 0.0f;
        if (off >= 0)
          for (int c = lane; c < a.channels; c += 64) {
            const float v = Ty::to_f32(a.x[off + c]);
            acc = fmaf(v, v, acc);
          }
        for (int m = 32; m > 0; m >>= 1) acc += __shfl_xor(acc, m);
        if (lane == 0) rrow[r] = rms_scale<Ty>(acc / static_cast<float>(a.channels), a.eps);
      }
    }
  }

  // Raw x tile [ROWS x D] into LDS (pad rows / columns read as zero).
  if (a.chan_contig && a.vec_ok) {
    constexpr int VPR = D / 8;
    for (int i = tid; i < ROWS * VPR; i += kThreads) {
      const int r = i / VPR, v = i % VPR;
      const int64_t off = rowoff[r];
      u32x4 val = {0u, 0u, 0u, 0u};
      if (off >= 0) val = *reinterpret_cast<const u32x4*>(a.x + off + qc * D + v * 8);
      *reinterpret_cast<u32x4*>(&xs[r * LDX + v * 8]) = val;
    }
  } else {
    for (int i = tid; i < ROWS * D; i += kThreads) {
      const int r = i / D, k = i % D;
      const int64_t off = rowoff[r];
      const int c = chx[k];
      xs[r * LDX + k] = (off >= 0 && c >= 0) ? a.x[off + c] : static_cast<uint16_t>(0);
    }
  }

  // Weight chunk 0 into LDS; later chunks are prefetched into registers one chunk ahead.
  const uint16_t* wsrc = a.packed + kHeadElems + static_cast<size_t>(qc) * NCH * CH_ELEMS;
  u32x4 pf[PF];
  auto prefetch = [&](int ec) {
    const u32x4* src = reinterpret_cast<const u32x4*>(wsrc + static_cast<size_t>(ec) * CH_ELEMS);
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < CH_VEC) pf[i] = src[idx];
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < CH_VEC) reinterpret_cast<u32x4*>(wb)[idx] = pf[i];
    }
  };
  prefetch(0);
  commit();

  const u32x2 fAu = reinterpret_cast<const u32x2*>(a.packed)[lane];
  const u32x2 fAv = reinterpret_cast<const u32x2*>(a.packed + kTokFragElems)[lane];
  const u32x2 fAo = reinterpret_cast<const u32x2*>(a.packed + 2 * kTokFragElems)[lane];
  __syncthreads();

  // Token side: P^T = T_norm^T . A^T for the wave's token groups, kept as bf16/fp16 B operands.
  const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  u32x4 Pu[TPW][KS], Pv[TPW][KS];
#pragma unroll
  for (int tg = 0; tg < TPW; ++tg) {
    const int row0 = (wave * TPW + tg) * kG;
    float rr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) rr[j] = rrow[row0 + 4 * h + j];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int k = mb * 16 + l16;
      const float w = wn[k];
      uint32_t e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint16_t raw = xs[(row0 + 4 * h + j) * LDX + k];
        if (fuse_norm) raw = Ty::from_f32(round_to<Ty>(Ty::to_f32(raw) * rr[j]) * w);
        e[j] = raw;
      }
      const u32x2 av = {e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
      const f32x4 pu = Ty::mma16(av, fAu, zero4);
      const f32x4 pv = Ty::mma16(av, fAv, zero4);
      Pu[tg][mb >> 1][(mb & 1) * 2 + 0] = pack2<Ty>(pu[0], pu[1]);
      Pu[tg][mb >> 1][(mb & 1) * 2 + 1] = pack2<Ty>(pu[2], pu[3]);
      Pv[tg][mb >> 1][(mb & 1) * 2 + 0] = pack2<Ty>(pv[0], pv[1]);
      Pv[tg][mb >> 1][(mb & 1) * 2 + 1] = pack2<Ty>(pv[2], pv[3]);
    }
  }

  // Channel side, streamed over 32-wide chunks of the expanded dimension.
  f32x4 W[TPW][MB];
#pragma unroll
  for (int tg = 0; tg < TPW; ++tg)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) W[tg][mb] = zero4;

  for (int ec = 0; ec < NCH; ++ec) {
    if (ec + 1 < NCH) prefetch(ec + 1);
    u32x4 Z[TPW];
#pragma unroll
    for (int eb = 0; eb < 2; ++eb) {
      f32x4 U[TPW], V[TPW];
#pragma unroll
      for (int tg = 0; tg < TPW; ++tg) U[tg] = V[tg] = zero4;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 fu = reinterpret_cast<const u32x4*>(wb + (eb * KS + ks) * kFragElems)[lane];
        const u32x4 fv = reinterpret_cast<const u32x4*>(wb + (FR_U + eb * KS + ks) * kFragElems)[lane];
#pragma unroll
        for (int tg = 0; tg < TPW; ++tg) {
          U[tg] = Ty::mma32(fu, Pu[tg][ks], U[tg]);
          V[tg] = Ty::mma32(fv, Pv[tg][ks], V[tg]);
        }
      }
#pragma unroll
      for (int tg = 0; tg < TPW; ++tg) {
        Z[tg][eb * 2 + 0] = pack2<Ty>(silu_gate(U[tg][0], V[tg][0]), silu_gate(U[tg][1], V[tg][1]));
        Z[tg][eb * 2 + 1] = pack2<Ty>(silu_gate(U[tg][2], V[tg][2]), silu_gate(U[tg][3], V[tg][3]));
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const u32x4 fo = reinterpret_cast<const u32x4*>(wb + (2 * FR_U + mb) * kFragElems)[lane];
#pragma unroll
      for (int tg = 0; tg < TPW; ++tg) W[tg][mb] = Ty::mma32(fo, Z[tg], W[tg][mb]);
    }
    if (ec + 1 < NCH) {
      __syncthreads();
      commit();
      __syncthreads();
    }
  }

  // Output side: W^T -> LDS (transpose), delta = A_o . W, LayerScale, residual, in place in xs.
  uint16_t* st = wst[wave];
#pragma unroll
  for (int tg = 0; tg < TPW; ++tg) {
    const int row0 = (wave * TPW + tg) * kG;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const u32x2 v = {pack2<Ty>(W[tg][mb][0], W[tg][mb][1]), pack2<Ty>(W[tg][mb][2], W[tg][mb][3])};
      *reinterpret_cast<u32x2*>(st + l16 * LDX + mb * 16 + 4 * h) = v;
    }
    wave_lds_sync();
#pragma unroll
    for (int nb = 0; nb < MB; ++nb) {
      const int k = nb * 16 + l16;
      uint32_t e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) e[j] = st[(4 * h + j) * LDX + k];
      const u32x2 bw = {e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
      const f32x4 dl = Ty::mma16(fAo, bw, zero4);
      const float g = gm[k];
      const bool col_ok = chx[k] >= 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = row0 + 4 * h + i;
        if (col_ok && rowoff[r] >= 0) {
          float v = round_to<Ty>(round_to<Ty>(dl[i]) * g);
          if (fuse_res) v = round_to<Ty>(Ty::to_f32(xs[r * LDX + k]) + v);
          xs[r * LDX + k] = Ty::from_f32(v);
        }
      }
    }
    wave_lds_sync();
  }
  __syncthreads();

  if (a.chan_contig && a.vec_ok) {
    constexpr int VPR = D / 8;
    for (int i = tid; i < ROWS * VPR; i += kThreads) {
      const int r = i / VPR, v = i % VPR;
      const int64_t off = rowoff[r];
      if (off >= 0)
        *reinterpret_cast<u32x4*>(a.out + off + qc * D + v * 8) =
            *reinterpret_cast<const u32x4*>(&xs[r * LDX + v * 8]);
    }
  } else {
    for (int i = tid; i < ROWS * D; i += kThreads) {
      const int r = i / D, k = i % D;
      const int64_t off = rowoff[r];
      const int c = chx[k];
      if (off >= 0 && c >= 0) a.out[off + c] = xs[r * LDX + k];
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
  void* packed;
  int32_t wdtype, q_c, d, rd;
  int64_t total;
};

__device__ __forceinline__ float load_f32(const void* p, int64_t i, int dtype) {
  if (dtype == OW_DTYPE_F32) return static_cast<const float*>(p)[i];
  const uint16_t u = static_cast<const uint16_t*>(p)[i];
  return dtype == OW_DTYPE_BF16 ? BF16::to_f32(u) : F16::to_f32(u);
}

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
    const int ks_n = p.d / 32, mb_n = p.d / 16, nch = p.rd / 32;
    const int fr_u = 2 * ks_n;
    const int64_t ch_elems = static_cast<int64_t>(2 * fr_u + mb_n) * kFragElems;
    int64_t rem = idx - kHeadElems;
    const int q = static_cast<int>(rem / (nch * ch_elems));
    rem -= static_cast<int64_t>(q) * nch * ch_elems;
    const int ec = static_cast<int>(rem / ch_elems);
    rem -= static_cast<int64_t>(ec) * ch_elems;
    const int fr = static_cast<int>(rem / kFragElems);
    const int e = static_cast<int>(rem % kFragElems);
    const int lane = e / 8, j = e % 8;
    const int l16 = lane & 15, h = lane >> 4;
    const int kk = 16 * (j / 4) + 4 * h + (j % 4);
    if (fr < 2 * fr_u) {
      // B_u^T / B_v^T operand: row e = 32ec + 16eb + l16, K = channel 32ks + kk.
      const int f = fr % fr_u;
      const int eb = f / ks_n, ks = f % ks_n;
      const int col = 32 * ec + 16 * eb + l16;
      const int c = 32 * ks + kk;
      const int64_t src = (static_cast<int64_t>(q) * p.d + c) * p.rd + col;
      val = load_f32(fr < fr_u ? p.b_u : p.b_v, src, p.wdtype);
    } else {
      // B_o^T operand: row = channel 16mb + l16, K = expanded index 32ec + kk.
      const int mb = fr - 2 * fr_u;
      const int c = 16 * mb + l16;
      const int ee = 32 * ec + kk;
      const int64_t src = (static_cast<int64_t>(q) * p.rd + ee) * p.d + c;
      val = load_f32(p.b_o, src, p.wdtype);
    }
  }
  static_cast<uint16_t*>(p.packed)[idx] = Ty::from_f32(val);
}

int64_t packed_elems(int32_t q_c, int32_t d, int32_t rd) {
  const int64_t per_chunk = static_cast<int64_t>(4 * (d / 32) + d / 16) * kFragElems;
  return kHeadElems + static_cast<int64_t>(q_c) * (rd / 32) * per_chunk;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return OW_OK;
  return fail(OW_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

template <class Ty, int D, int RD>
int launch_fwd(const FwdArgs& a, hipStream_t stream) {
  constexpr int TPW = 2;
  constexpr int R = kWaves * TPW;
  FwdArgs args = a;
  const int64_t groups = static_cast<int64_t>(a.batch) * a.q_s;
  const int64_t chunks = (groups + R - 1) / R;
  const int64_t nwg = chunks * a.q_c;
  if (nwg == 0) return OW_OK;
  if (nwg > 0x7fffffff) return fail(OW_ERR_UNSUPPORTED, "grid too large (%lld workgroups)", (long long)nwg);
  args.n_chunks = static_cast<int32_t>(chunks);
  hipLaunchKernelGGL((bigemm_fwd_kernel<Ty, D, RD, TPW>), dim3(static_cast<unsigned>(nwg)), dim3(kThreads), 0,
                     stream, args);
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

int ow_pack_weights(const void* a_u, const void* a_v, const void* a_o, const void* b_u, const void* b_v,
                    const void* b_o, int32_t weight_dtype, int32_t g, int32_t q_c, int32_t d, int32_t rd,
                    int32_t compute_dtype, void* packed, void* stream) {
  OW_CHECK_ARG(a_u && a_v && a_o && b_u && b_v && b_o && packed, "weight or output pointer is NULL");
  OW_CHECK_ARG(weight_dtype >= OW_DTYPE_F32 && weight_dtype <= OW_DTYPE_F16, "unknown weight dtype %d", weight_dtype);
  OW_CHECK_SUPPORTED(g == ow::kG, "unsupported spatial tile g=%d; expected 16", g);
  OW_CHECK_ARG(q_c >= 1, "q_c must be >= 1 (got %d)", q_c);
  OW_CHECK_SUPPORTED((d == 64 || d == 128) && (rd == 128 || rd == 256),
                     "unsupported channel tile d=%d / expanded dim rd=%d", d, rd);
  OW_CHECK_SUPPORTED(compute_dtype == OW_DTYPE_BF16 || compute_dtype == OW_DTYPE_F16,
                     "unsupported compute dtype %d", compute_dtype);
  ow::PackArgs p{a_u, a_v, a_o, b_u, b_v, b_o, packed, weight_dtype, q_c, d, rd, ow::packed_elems(q_c, d, rd)};
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

int ow_bigemm_fwd(const void* x, void* out, const float* norm_weight, float eps, const float* gamma,
                  const void* packed, size_t packed_bytes, const int32_t* token_index,
                  const int32_t* channel_index, const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype,
                  int32_t flags, void* stream) {
  int32_t q_s = 0, q_c = 0;
  if (int rc = ow_plan_dims(plan, &q_s, &q_c)) return rc;
  OW_CHECK_ARG(batch >= 0, "batch must be >= 0 (got %d)", batch);
  OW_CHECK_ARG(x && out && gamma && packed && token_index && channel_index, "tensor pointer is NULL");
  OW_CHECK_ARG(x != out, "out must not alias x");
  OW_CHECK_ARG(!(flags & OW_FUSE_NORM) || norm_weight, "OW_FUSE_NORM needs norm_weight");
  OW_CHECK_ARG((flags & ~(OW_FUSE_NORM | OW_FUSE_RESIDUAL)) == 0, "unknown flags 0x%x", flags);
  OW_CHECK_SUPPORTED(plan->spatial_tile == ow::kG, "unsupported spatial tile g=%d; expected 16", plan->spatial_tile);
  OW_CHECK_SUPPORTED(dtype == OW_DTYPE_BF16 || dtype == OW_DTYPE_F16,
                     "unsupported dtype %d; expected bf16 or f16", dtype);
  const int32_t n = plan->height * plan->width, c = plan->channels, d = plan->channel_tile;
  OW_CHECK_ARG(static_cast<int64_t>(batch) * n * c < (int64_t(1) << 40), "tensor too large");
  const size_t want = ow_packed_weight_bytes(q_c, d, rd, dtype);
  OW_CHECK_ARG(want != 0 && packed_bytes == want,
               "packed weights hold %zu bytes; q_c=%d d=%d rd=%d needs %zu", packed_bytes, q_c, d, rd, want);
  ow::FwdArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.out = static_cast<uint16_t*>(out);
  a.norm_w = norm_weight;
  a.gamma = gamma;
  a.packed = static_cast<const uint16_t*>(packed);
  a.tok = token_index;
  a.chan = channel_index;
  a.batch = batch;
  a.n_tok = n;
  a.channels = c;
  a.q_s = q_s;
  a.q_c = q_c;
  a.flags = flags;
  a.eps = eps;
  a.chan_contig = (c % d == 0) && (plan->radix_level == 0 || q_c <= 1);
  a.vec_ok = (c % 8 == 0) && ow::aligned16(x) && ow::aligned16(out);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rc = dtype == OW_DTYPE_BF16 ? ow::dispatch_fwd<ow::BF16>(a, d, rd, s)
                                        : ow::dispatch_fwd<ow::F16>(a, d, rd, s);
  if (rc == OW_OK) ow::clear_error();
  return rc;
}

}  // extern "C"
