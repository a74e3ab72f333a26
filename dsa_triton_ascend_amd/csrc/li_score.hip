// Lightning-indexer score kernel for gfx950.
//
// Computes, per packed query row r (batch b, position s1) and key head n2,
//   score[s2] = sum_{g<G} relu(q[r, n2*G+g, :] . k[b, s2, n2, :]) * w[r, n2*G+g]
// for the visible key prefix s2 < L(s1) and writes it quantised (bf16 RNE or
// fp16) -- the arithmetic of _lightning_indexer_score_kernel
// (lightning_indexer_triton.py:180-284) and of the golden
// (lightning_indexer_numpy.py:75-92), whose quantisation happens before top-k.
//
// Mapping onto CDNA4:
//  * one wave owns one query row; the row's G heads are the MFMA M dimension
//    (MT tiles of 32 heads), keys are N (32 per MFMA), D is the contraction:
//    v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation;
//  * the row's Q fragments stay in VGPRs for the whole key sweep (MT <= 2, MT*D <= 512),
//    otherwise they are re-read from L2 per key tile;
//  * a work-group = NW waves = NW consecutive query rows of one (batch, n2);
//    they share each 64-key K tile, staged global -> VGPR -> LDS with a
//    one-tile register prefetch and two LDS buffers (one barrier per tile);
//    LDS rows are padded by 16 B so the 16-byte B-fragment reads are
//    conflict-free;
//  * per tile a wave issues its B-fragment reads ahead of the MFMAs and keeps
//    one accumulator set per 32-key subtile, so the epilogue of one subtile can
//    overlap the MFMAs of the next;
//  * the epilogue is fused: relu(acc) * w[head] summed over the 16 heads a lane
//    holds and the MT tiles (four independent partial sums), then one
//    cross-lane add (lanes l and l^32) gives the per-key score; fully causal-
//    masked tiles are never loaded or computed;
//  * row blocks are issued heaviest-first (largest s1 first) to flatten the
//    causal triangle's tail.
#include "dsa_common.hpp"

namespace dsa {

namespace {

#ifndef DSA_LI_NW
#define DSA_LI_NW 8
#endif
#ifndef DSA_LI_BN
#define DSA_LI_BN 64
#endif
constexpr int NW = DSA_LI_NW;  // waves (= query rows) per work-group

template <int D> struct LiTile {
  static constexpr int BN = D <= 128 ? DSA_LI_BN : 32;  // keys per LDS tile
  static constexpr int PITCH = D + 8;                  // uint16 elements per LDS key row
  static constexpr int CHUNKS = BN * D / 8;            // 16-byte chunks per tile
  static constexpr int CPT = (CHUNKS + NW * 64 - 1) / (NW * 64);   // chunks per thread
};

__device__ __forceinline__ float load_w(const void* w, int wdt, int64_t i) {
  if (wdt == DSA_DTYPE_F32) return reinterpret_cast<const float*>(w)[i];
  uint16_t h = reinterpret_cast<const uint16_t*>(w)[i];
  return wdt == DSA_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

__device__ __forceinline__ int visible_len(int s1, int aq, int ak, int S2, int mode) {
  int L;
  if (mode == 3) {
    L = ak - aq + s1 + 1;
    L = L < 0 ? 0 : L;
    L = L < S2 ? L : S2;
    L = L < ak ? L : ak;
  } else {
    L = ak < S2 ? ak : S2;
  }
  return L < 0 ? 0 : L;
}

template <int IO, int D, int MT>
__global__ __launch_bounds__(NW * 64) void li_score_kernel(LiScoreArgs a) {
  using T = LiTile<D>;
  constexpr int KK = D / 16;                 // MFMA k-steps
  constexpr int NSUB = T::BN / 32;           // 32-key subtiles per tile
  constexpr bool QREG = MT <= 2 && MT * D <= 512;   // Q fragments resident in VGPRs
  __shared__ __attribute__((aligned(16))) uint16_t kt[2][T::BN * T::PITCH];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int b = blockIdx.z;
  const int n2 = blockIdx.y;
  const int rb = gridDim.x - 1 - blockIdx.x;  // heaviest row block first
  const int G = a.n1 / a.n2;

  const int rows_b = a.row_start[b + 1] - a.row_start[b];
  const int aq = a.act_q[b], ak = a.act_k[b];
  const int nrows = rows_b < aq ? rows_b : aq;     // rows that produce scores
  const int s1_0 = rb * NW;
  if (s1_0 >= nrows) return;
  const int s1_last = (s1_0 + NW - 1 < nrows ? s1_0 + NW - 1 : nrows - 1);
  const int L_blk = visible_len(s1_last, aq, ak, a.s2, a.sparse_mode);  // monotone in s1
  if (L_blk <= 0) return;

  const int s1 = s1_0 + wave;
  const bool row_ok = s1 < nrows;
  const int L_row = row_ok ? visible_len(s1, aq, ak, a.s2, a.sparse_mode) : 0;
  const int64_t r = (int64_t)a.row_start[b] + (row_ok ? s1 : s1_0);

  const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + (r * a.n1 + (int64_t)n2 * G) * D;
  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(a.k) +
                          ((int64_t)a.key_start[b] * a.n2 + n2) * D;
  const int64_t kstride = (int64_t)a.n2 * D;

  // ---- K tile staging (started first so its latency overlaps the Q / w loads)
  const int ntiles = (L_blk + T::BN - 1) / T::BN;
  uint4 pre[T::CPT];
  auto fetch = [&](int tile) {
#pragma unroll
    for (int c = 0; c < T::CPT; ++c) {
      const int ch = threadIdx.x + c * NW * 64;
      const int key = ch / (D / 8), off = (ch % (D / 8)) * 8;
      const int s2 = tile * T::BN + key;
      pre[c] = (ch < T::CHUNKS && s2 < L_blk) ? ldg16(kbase + (int64_t)s2 * kstride + off)
                                              : make_uint4(0, 0, 0, 0);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int c = 0; c < T::CPT; ++c) {
      const int ch = threadIdx.x + c * NW * 64;
      if (ch < T::CHUNKS) {
        const int key = ch / (D / 8), off = (ch % (D / 8)) * 8;
        *reinterpret_cast<uint4*>(&kt[buf][key * T::PITCH + off]) = pre[c];
      }
    }
  };
  fetch(0);

  // ---- per-row operands: Q fragments (A) and head weights
  uint4 qf[QREG ? MT : 1][QREG ? KK : 1];
  if constexpr (QREG) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 32 + (lane & 31);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        qf[mt][kk] = (row_ok && m < G) ? ldg16(qrow + (int64_t)m * D + kk * 16 + (lane >> 5) * 8)
                                       : make_uint4(0, 0, 0, 0);
    }
  }
  // weights: one coalesced load per lane (head = lane + 64 j), then each lane
  // gathers the 16 heads it holds in the MFMA output layout with lane shuffles
  float wv[MT][16];
  {
    constexpr int WJ = (MT * 32 + 63) / 64;
    float wl[WJ];
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
      const int h = lane + 64 * j;
      wl[j] = (row_ok && h < G) ? load_w(a.w, a.wdt, r * a.n1 + (int64_t)n2 * G + h) : 0.f;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int h = mt * 32 + m32_row(i, lane);
        const float v = __shfl(wl[(mt * 32) / 64], h & 63);
        wv[mt][i] = v;
      }
  }

  uint16_t* srow = a.scores + (r * a.n2 + n2) * a.ld;

  // ---- main loop, software-pipelined by 32-key subtile: the MFMAs of subtile
  // j are interleaved with the relu*w epilogue of subtile j-1 (ping-pong
  // accumulators), so the wave's VALU work co-executes with its MFMAs.
  f32x16 acc[2][MT];
  int pend_key0 = -1;   // first key of the subtile whose epilogue is pending (-1: none)

  auto zero = [&](f32x16(&c)[MT]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) c[mt][i] = 0.f;
  };
  auto finish = [&](float (&p4)[4], int key0) {
    float p = (p4[0] + p4[1]) + (p4[2] + p4[3]);
    p += __shfl_xor(p, 32);
    const int s2 = key0 + (lane & 31);
    if (lane < 32 && s2 < L_row) srow[s2] = from_f32<IO>(p);
  };
  // one subtile: MFMAs into `cur` from the LDS rows at `bp`; epilogue of `prev` interleaved
  auto step = [&](f32x16(&cur)[MT], f32x16(&prev)[MT], const uint16_t* bp, bool has_prev, int prev_key0) {
    constexpr int KC = KK < 8 ? KK : 8;
    constexpr int EPK = (MT * 16 + KK - 1) / KK;   // epilogue elements per k-step
    float p4[4] = {0.f, 0.f, 0.f, 0.f};
    zero(cur);
#pragma unroll
    for (int k0 = 0; k0 < KK; k0 += KC) {
      uint4 bf[KC];
#pragma unroll
      for (int j = 0; j < KC; ++j) bf[j] = *reinterpret_cast<const uint4*>(bp + (k0 + j) * 16);
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        const int kk = k0 + j;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          uint4 af;
          if constexpr (QREG) {
            af = qf[mt][kk];
          } else {
            const int m = mt * 32 + (lane & 31);
            af = (row_ok && m < G) ? ldg16(qrow + (int64_t)m * D + kk * 16 + (lane >> 5) * 8)
                                   : make_uint4(0, 0, 0, 0);
          }
          cur[mt] = Mfma<IO>::m32(af, bf[j], cur[mt]);
        }
        if (has_prev) {
#pragma unroll
          for (int q = 0; q < EPK; ++q) {
            const int e = kk * EPK + q;
            if (e < MT * 16) p4[e & 3] += fmaxf(prev[e >> 4][e & 15], 0.f) * wv[e >> 4][e & 15];
          }
        }
      }
    }
    if (has_prev) finish(p4, prev_key0);
  };
  auto drain = [&](f32x16(&prev)[MT], int key0) {
    float p4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < MT * 16; ++e) p4[e & 3] += fmaxf(prev[e >> 4][e & 15], 0.f) * wv[e >> 4][e & 15];
    finish(p4, key0);
  };

  stash(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) fetch(t + 1);
    const uint16_t* bp0 = &kt[buf][(lane & 31) * T::PITCH + (lane >> 5) * 8];
    if (t * T::BN < L_row) {  // wave-uniform: this row sees part of the tile
      if constexpr (NSUB % 2 == 0) {
#pragma unroll
        for (int sub = 0; sub < NSUB; sub += 2) {
          step(acc[0], acc[1], bp0 + sub * 32 * T::PITCH, sub > 0 || pend_key0 >= 0,
               sub > 0 ? t * T::BN + (sub - 1) * 32 : pend_key0);
          step(acc[1], acc[0], bp0 + (sub + 1) * 32 * T::PITCH, true, t * T::BN + sub * 32);
        }
        pend_key0 = t * T::BN + (NSUB - 1) * 32;
      } else {
        step(acc[0], acc[1], bp0, false, 0);
        drain(acc[0], t * T::BN);
      }
    } else if (pend_key0 >= 0) {
      drain(acc[1], pend_key0);
      pend_key0 = -1;
    }
    if (t + 1 < ntiles) stash(buf ^ 1);
    __syncthreads();
  }
  if (pend_key0 >= 0) drain(acc[1], pend_key0);
}

template <int IO, int D>
hipError_t launch_d(const LiScoreArgs& a, hipStream_t s, int MT) {
  dim3 grid((a.max_rows_per_batch + NW - 1) / NW, a.n2, a.batch), block(NW * 64);
  switch (MT) {
    case 1: hipLaunchKernelGGL((li_score_kernel<IO, D, 1>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((li_score_kernel<IO, D, 2>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((li_score_kernel<IO, D, 4>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

template <int IO>
hipError_t launch_io(const LiScoreArgs& a, hipStream_t s, int MT) {
  switch (a.d) {
    case 64: return launch_d<IO, 64>(a, s, MT);
    case 96: return launch_d<IO, 96>(a, s, MT);
    case 128: return launch_d<IO, 128>(a, s, MT);
    case 256: return launch_d<IO, 256>(a, s, MT);
    case 512: return launch_d<IO, 512>(a, s, MT);
  }
  return hipErrorInvalidValue;
}

}  // namespace

}  // namespace dsa

bool li_score_supported_d(int d) { return d == 64 || d == 96 || d == 128 || d == 256 || d == 512; }

hipError_t launch_li_score(const LiScoreArgs& a, hipStream_t s) {
  const int G = a.n1 / a.n2;
  const int MT = G <= 32 ? 1 : (G <= 64 ? 2 : 4);
  if (a.max_rows_per_batch <= 0 || a.total_rows <= 0) return hipSuccess;
  return a.io == dsa::IO_BF16 ? dsa::launch_io<dsa::IO_BF16>(a, s, MT)
                              : dsa::launch_io<dsa::IO_F16>(a, s, MT);
}
