// Sparse flash attention backward (MLA-absorb, N2 = 1) for gfx950.
//
// Semantics: sparse_flash_attention_grad_numpy.py:34-143 (the golden), the
// inputs and outputs of sparse_flash_attention_grad_triton.py:498-677. Per
// query row and head, with the forward's output O and softmax stats:
//   P  = exp(score - sm_max) / sm_sum,  score = (q . k + q_rope . k_rope) * scale
//   dS = P * (dO . k_nope - dO . O) * scale
//   d_query | d_query_rope = dS @ [k_nope | k_rope]          (per row)
//   d_key | d_key_rope    += dS^T @ [q_nope | q_rope]        (scatter over tokens)
//   d_value               += P^T @ dO                        (scatter over tokens)
//
// Launches:
//  1. the forward's token-list kernels (the golden's gather order, physical key
//     rows), so both passes select exactly the same tokens;
//  2. sfa_bwd_zero_kernel -- clears the fp32 d_key / d_key_rope / d_value
//     accumulators in the workspace;
//  3. sfa_bwd_kernel -- one work-group (4 waves) per (query row, block of 32
//     heads). Q | Q rope and dO of the block sit in LDS for the whole row; the
//     row's tokens are processed in tiles of 32 gathered [D | Dr] rows:
//       * S^T = K Q^T and dP^T = K_nope dO^T on v_mfma_f32_32x32x16 (tokens as
//         M, heads as N), their k-ranges split over the four waves and summed
//         through LDS;
//       * P and dS (fp32, then the io dtype) go to LDS as [head][token];
//       * each wave then owns a quarter of the 32-column blocks of
//         dQ (accumulated in registers over the row), of the tile's
//         dK = dS^T [Q | Q rope] and of its dV = P^T dO; the operands whose K is
//         the token or head index are read with ds_read_b64_tr_b16 from the
//         row-major LDS arrays;
//       * the dK / dV blocks are added to fp32 accumulators at the tokens'
//         physical rows with global fp32 atomics (a key row selected by several
//         query rows gets all their contributions; the order of the additions,
//         and so the last bits, may differ from run to run -- the reference's
//         contract, deterministic=False, sparse_flash_attention_grad_triton.py:550);
//  4. sfa_bwd_finish_kernel -- converts the accumulators to the io dtype.
#include <climits>

#include "dsa_common.hpp"

namespace dsa {
namespace {

constexpr int BDR = 64;     // rope width
constexpr int BH = 32;      // heads per work-group
constexpr int BT = 32;      // tokens per tile
constexpr int BWV = 4;      // waves per work-group
constexpr float BLOG2E = 1.4426950408889634f;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

template <int D> struct BCfg {
  static constexpr int DT = D + BDR;                   // [nope | rope] width
  static constexpr int QP = DT + 8;                    // Q / K row pitch: odd count of 16-byte units
  static constexpr int OP = D + 8;                     // dO row pitch
  static constexpr int PP = BT + 8;                    // P / dS row pitch
  static constexpr int NBQ = DT / 32;                  // 32-column blocks of dQ and dK
  static constexpr int NBV = D / 32;                   // of dV
  static constexpr int JQ = (NBQ + BWV - 1) / BWV;     // dQ blocks per wave, at most
  static constexpr int KS_S = DT / 16;                 // k-steps of S^T
  static constexpr int KS_P = D / 16;                  // of dP^T
  static_assert(KS_S % 2 == 0 && KS_P % 2 == 0, "k-ranges split in halves");
};

// MFMA 32x32x16 operand whose K runs down the rows of a row-major 16-bit LDS
// array X (pitch in elements): lane l receives X[k0 + 8 (l / 32) + j][c0 + l % 32],
// j = 0..7, from two transposed 8-byte reads (rows k and k + 4 of its group).
__device__ __forceinline__ uint4 tr_frag(const uint16_t* X, int pitch, int c0, int k0, int lane) {
  const int g16 = lane >> 4, c16 = lane & 15;
  const int col = c0 + (g16 & 1) * 16 + 4 * (c16 & 3);
  const int k = k0 + (g16 >> 1) * 8 + (c16 >> 2);
  const uint2 lo = ds_read_tr(X + k * pitch + col);
  const uint2 hi = ds_read_tr(X + (k + 4) * pitch + col);
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

struct BwdAcc {
  float* dk;    // [key_rows, D]
  float* dkr;   // [key_rows, Dr]
  float* dv;    // [key_rows, D]
};

template <int IO, int D>
__global__ __launch_bounds__(BWV * 64) void sfa_bwd_kernel(SfaBwdArgs a, SfaTokenLists tl, BwdAcc acc) {
  using C = BCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t Qs[BH * C::QP];    // [head][nope | rope]
  __shared__ __attribute__((aligned(16))) uint16_t Ks[BT * C::QP];    // [token][nope | rope]
  __shared__ __attribute__((aligned(16))) uint16_t dOs[BH * C::OP];   // [head][D]
  __shared__ __attribute__((aligned(16))) uint16_t Ps[BH * C::PP];    // [head][token]
  __shared__ __attribute__((aligned(16))) uint16_t dSs[BH * C::PP];   // [head][token]
  __shared__ float part[BWV][16][64];   // S^T / dP^T k-range partials, MFMA layout
  __shared__ int s_tok[BT];
  __shared__ float s_m[BH], s_il[BH], s_dl[BH];

  const SfaArgs& f = a.f;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = f.total_rows - 1 - (int)blockIdx.x;   // long (late causal) rows first
  const int n1 = f.n1;
  const int h0 = blockIdx.y * BH;
  const int hn = n1 - h0 < BH ? n1 - h0 : BH;          // heads of this block
  const int krows = f.key_rows < INT_MAX ? (int)f.key_rows : INT_MAX;
  const int ntok = tl.counts[r];
  const int32_t* toks = tl.tokens + (int64_t)r * tl.tstride;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(f.k);
  const uint16_t* krb = reinterpret_cast<const uint16_t*>(f.kr);
  const uint4 z4 = make_uint4(0, 0, 0, 0);

  // ---- the block's Q | Q rope and dO (rows past the heads are zero), stats
  {
    const uint16_t* qb = reinterpret_cast<const uint16_t*>(f.q);
    const uint16_t* qrb = reinterpret_cast<const uint16_t*>(f.qr);
    const uint16_t* gob = reinterpret_cast<const uint16_t*>(a.d_out);
    for (int i = tid; i < BH * (C::DT / 8); i += BWV * 64) {
      const int h = i / (C::DT / 8), c = (i % (C::DT / 8)) * 8;
      uint4 v = z4;
      if (h < hn) {
        const int64_t hr = (int64_t)r * n1 + h0 + h;
        v = c < D ? ldg16(qb + hr * D + c) : ldg16(qrb + hr * BDR + (c - D));
      }
      *reinterpret_cast<uint4*>(&Qs[h * C::QP + c]) = v;
    }
    for (int i = tid; i < BH * (D / 8); i += BWV * 64) {
      const int h = i / (D / 8), c = (i % (D / 8)) * 8;
      const uint4 v = h < hn ? ldg16(gob + ((int64_t)r * n1 + h0 + h) * D + c) : z4;
      *reinterpret_cast<uint4*>(&dOs[h * C::OP + c]) = v;
    }
    // delta = dO . O (fp32) per head: 8 threads per head, D/8 columns each
    const uint16_t* ob = reinterpret_cast<const uint16_t*>(a.out);
    const int h = tid >> 3, part8 = tid & 7;
    float dl = 0.f;
    if (h < hn) {
      const int64_t hr = (int64_t)r * n1 + h0 + h;
      for (int c = part8 * 8; c < D; c += 64) {
        const uint4 o = ldg16(ob + hr * D + c), g = ldg16(gob + hr * D + c);
        const uint32_t ow[4] = {o.x, o.y, o.z, o.w}, gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dl += to_f32<IO>((uint16_t)(ow[j] & 0xFFFFu)) * to_f32<IO>((uint16_t)(gw[j] & 0xFFFFu));
          dl += to_f32<IO>((uint16_t)(ow[j] >> 16)) * to_f32<IO>((uint16_t)(gw[j] >> 16));
        }
      }
    }
    dl += __shfl_xor(dl, 1);
    dl += __shfl_xor(dl, 2);
    dl += __shfl_xor(dl, 4);
    if (part8 == 0 && h < BH) {
      float m = 0.f, il = 0.f;
      if (h < hn) {
        const int64_t hr = (int64_t)r * n1 + h0 + h;
        m = a.sm_max[hr];
        const float l = a.sm_sum[hr];
        il = l > 0.f ? 1.f / l : 0.f;
      }
      s_m[h] = m * BLOG2E;
      s_il[h] = il;
      s_dl[h] = h < hn ? dl : 0.f;
    }
  }

  f32x16 dq[C::JQ];
#pragma unroll
  for (int jj = 0; jj < C::JQ; ++jj)
#pragma unroll
    for (int i = 0; i < 16; ++i) dq[jj][i] = 0.f;
  const float sl2 = f.scale * BLOG2E;

  for (int t0 = 0; t0 < ntok; t0 += BT) {
    const int nv = ntok - t0 < BT ? ntok - t0 : BT;
    // ---- gather the tile's [nope | rope] rows; rows outside the key tensors and
    // slots past the list are zero
    for (int i = tid; i < BT * (C::DT / 8); i += BWV * 64) {
      const int t = i / (C::DT / 8), c = (i % (C::DT / 8)) * 8;
      const int p = t < nv ? toks[t0 + t] : -1;
      uint4 v = z4;
      if ((uint32_t)p < (uint32_t)krows)
        v = c < D ? ldg16(kb + (int64_t)p * D + c) : ldg16(krb + (int64_t)p * BDR + (c - D));
      *reinterpret_cast<uint4*>(&Ks[t * C::QP + c]) = v;
    }
    if (tid < BT) {
      const int p = tid < nv ? toks[t0 + tid] : -1;
      s_tok[tid] = (uint32_t)p < (uint32_t)krows ? p : -1;
    }
    __syncthreads();

    // ---- S^T (waves 0, 1: halves of the [nope | rope] k-range) and dP^T (waves 2,
    // 3: halves of the nope range), tokens as M, heads as N
    {
      const bool is_s = wave < 2;
      const int nks = is_s ? C::KS_S / 2 : C::KS_P / 2;
      const int ks0 = (wave & 1) * nks;
      const uint16_t* arow = Ks + (lane & 31) * C::QP + (lane >> 5) * 8 + ks0 * 16;
      const uint16_t* brow = (is_s ? Qs + (lane & 31) * C::QP : dOs + (lane & 31) * C::OP) + (lane >> 5) * 8 + ks0 * 16;
      f32x16 s = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int ks = 0; ks < nks; ++ks)
        s = Mfma<IO>::m32(*reinterpret_cast<const uint4*>(arow + ks * 16),
                          *reinterpret_cast<const uint4*>(brow + ks * 16), s);
#pragma unroll
      for (int i = 0; i < 16; ++i) part[wave][i][lane] = s[i];
    }
    __syncthreads();

    // ---- P and dS of the tile (fp32, stored in the io dtype as [head][token])
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = wave * 4 + j;
      const int tk = m32_row(i, lane), h = lane & 31;
      const float sv = part[0][i][lane] + part[1][i][lane];
      const float dp = part[2][i][lane] + part[3][i][lane];
      float p = 0.f, ds = 0.f;
      if (tk < nv && h < hn) {
        p = __builtin_amdgcn_exp2f(sv * sl2 - s_m[h]) * s_il[h];
        ds = p * (dp - s_dl[h]) * f.scale;
      }
      Ps[h * C::PP + tk] = from_f32<IO>(p);
      dSs[h * C::PP + tk] = from_f32<IO>(ds);
    }
    __syncthreads();

    // ---- dQ[head, col] += dS[head, token] K[token, col]   (this wave's column blocks)
#pragma unroll
    for (int jj = 0; jj < C::JQ; ++jj) {
      const int j = wave + BWV * jj;
      if (j < C::NBQ) {
#pragma unroll
        for (int kq = 0; kq < BT / 16; ++kq) {
          const uint4 av = *reinterpret_cast<const uint4*>(dSs + (lane & 31) * C::PP + kq * 16 + (lane >> 5) * 8);
          dq[jj] = Mfma<IO>::m32(av, tr_frag(Ks, C::QP, 32 * j, kq * 16, lane), dq[jj]);
        }
      }
    }
    // ---- dK[token, col] = dS^T Q and dV[token, col] = P^T dO, added at the
    // tokens' key rows (fp32 atomics, coalesced along the 32 columns of a block)
#pragma unroll
    for (int jj = 0; jj < C::JQ; ++jj) {
      const int j = wave + BWV * jj;
      if (j < C::NBQ) {
        f32x16 c = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kq = 0; kq < BH / 16; ++kq)
          c = Mfma<IO>::m32(tr_frag(dSs, C::PP, 0, kq * 16, lane), tr_frag(Qs, C::QP, 32 * j, kq * 16, lane), c);
        const int col = 32 * j + (lane & 31);
        float* dst = col < D ? acc.dk + col : acc.dkr + (col - D);
        const int ld = col < D ? D : BDR;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int p = s_tok[m32_row(i, lane)];
          if (p >= 0) unsafeAtomicAdd(dst + (int64_t)p * ld, c[i]);
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < (C::NBV + BWV - 1) / BWV; ++jj) {
      const int j = wave + BWV * jj;
      if (j < C::NBV) {
        f32x16 c = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kq = 0; kq < BH / 16; ++kq)
          c = Mfma<IO>::m32(tr_frag(Ps, C::PP, 0, kq * 16, lane), tr_frag(dOs, C::OP, 32 * j, kq * 16, lane), c);
        float* dst = acc.dv + 32 * j + (lane & 31);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int p = s_tok[m32_row(i, lane)];
          if (p >= 0) unsafeAtomicAdd(dst + (int64_t)p * D, c[i]);
        }
      }
    }
    __syncthreads();   // the next tile overwrites Ks, Ps, dSs and s_tok
  }

  // ---- d_query | d_query_rope of the block's heads (zeros for rows without tokens)
  uint16_t* dqo = reinterpret_cast<uint16_t*>(a.dq);
  uint16_t* dqro = reinterpret_cast<uint16_t*>(a.dqr);
#pragma unroll
  for (int jj = 0; jj < C::JQ; ++jj) {
    const int j = wave + BWV * jj;
    if (j < C::NBQ) {
      const int col = 32 * j + (lane & 31);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int h = m32_row(i, lane);
        if (h < hn) {
          const int64_t hr = (int64_t)r * n1 + h0 + h;
          const uint16_t v = from_f32<IO>(dq[jj][i]);
          if (col < D) dqo[hr * D + col] = v;
          else dqro[hr * BDR + (col - D)] = v;
        }
      }
    }
  }
}

__global__ void sfa_bwd_zero_kernel(float4* p, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

// fp32 accumulator -> io dtype, 4 elements per step (every length is a multiple of 4)
template <int IO>
__global__ void sfa_bwd_finish_kernel(const float4* src, uint2* dst, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    const float4 v = src[i];
    dst[i] = make_uint2(pack2<IO>(v.x, v.y), pack2<IO>(v.z, v.w));
  }
}

template <int IO>
hipError_t launch_bwd_io(const SfaBwdArgs& a, const SfaTokenLists& tl, BwdAcc acc, hipStream_t s) {
  const SfaArgs& f = a.f;
  if (f.total_rows > 0) {
    const dim3 grid(f.total_rows, (f.n1 + BH - 1) / BH);
    switch (f.d) {
      case 128: hipLaunchKernelGGL((sfa_bwd_kernel<IO, 128>), grid, dim3(BWV * 64), 0, s, a, tl, acc); break;
      case 256: hipLaunchKernelGGL((sfa_bwd_kernel<IO, 256>), grid, dim3(BWV * 64), 0, s, a, tl, acc); break;
      case 512: hipLaunchKernelGGL((sfa_bwd_kernel<IO, 512>), grid, dim3(BWV * 64), 0, s, a, tl, acc); break;
      default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int64_t kr = f.key_rows;
  const struct { const float* src; void* dst; int64_t n; } outs[3] = {
      {acc.dk, a.dk, kr * f.d}, {acc.dkr, a.dkr, kr * BDR}, {acc.dv, a.dv, kr * f.d}};
  for (const auto& o : outs) {
    if (o.n == 0) continue;
    const int64_t n4 = o.n / 4;
    const int blocks = (int)((n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096);
    hipLaunchKernelGGL((sfa_bwd_finish_kernel<IO>), dim3(blocks), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(o.src), reinterpret_cast<uint2*>(o.dst), n4);
  }
  return hipGetLastError();
}

}  // namespace
}  // namespace dsa

size_t sfa_bwd_workspace_bytes(int total_rows, int n1, int topk, int sbs, int64_t key_rows, int d) {
  (void)n1;
  size_t off = dsa::align256(sfa_token_ws_bytes(total_rows > 0 ? total_rows : 1, topk, sbs));
  off += dsa::align256((size_t)key_rows * d * 4);
  off += dsa::align256((size_t)key_rows * dsa::BDR * 4);
  off += dsa::align256((size_t)key_rows * d * 4);
  return off;
}

hipError_t launch_sfa_bwd(const SfaBwdArgs& a, hipStream_t s) {
  const SfaArgs& f = a.f;
  char* base = reinterpret_cast<char*>(f.ws);
  SfaTokenLists tl{};
  hipError_t e = launch_sfa_token_lists(f, base, &tl, s);
  if (e != hipSuccess) return e;
  size_t off = dsa::align256(sfa_token_ws_bytes(f.total_rows > 0 ? f.total_rows : 1, f.topk, f.sbs));
  dsa::BwdAcc acc;
  acc.dk = reinterpret_cast<float*>(base + off);
  off += dsa::align256((size_t)f.key_rows * f.d * 4);
  acc.dkr = reinterpret_cast<float*>(base + off);
  off += dsa::align256((size_t)f.key_rows * dsa::BDR * 4);
  acc.dv = reinterpret_cast<float*>(base + off);
  off += dsa::align256((size_t)f.key_rows * f.d * 4);
  // the three accumulators are contiguous up to the 256-byte padding: clear the span
  const int64_t n4 = (int64_t)((off - (reinterpret_cast<char*>(acc.dk) - base)) / 16);
  if (n4 > 0) {
    const int blocks = (int)((n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096);
    hipLaunchKernelGGL(dsa::sfa_bwd_zero_kernel, dim3(blocks), dim3(256), 0, s,
                       reinterpret_cast<float4*>(acc.dk), n4);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return f.io == dsa::IO_BF16 ? dsa::launch_bwd_io<dsa::IO_BF16>(a, tl, acc, s)
                              : dsa::launch_bwd_io<dsa::IO_F16>(a, tl, acc, s);
}
