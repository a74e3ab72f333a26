// Sparse flash attention forward (MLA-absorb, N2 = 1) for gfx950.
//
// Semantics: sparse_flash_attention_numpy.py:38-160 (the golden) with the
// layouts of sparse_flash_attention_triton.py:1353-1450.
//
// Two kernels:
//  1. sfa_tokens_kernel  -- one work-group per packed query row: applies the
//     row-skip rules and the golden's gatherKV scan (first
//     min(count, ceil(threshold/bs)) ids, stop at the first -1, expand id to
//     [id*bs, min(id*bs+bs, act_k, threshold))), and writes the row's token
//     list as PHYSICAL key rows (key_start offset, or the PA block-table
//     lookup; a -1 block gives -1 = zero row) into the workspace.  This is the
//     work the reference does with _expand_block_indices / _pa_to_bsnd on the
//     host plus its masked loads (:1012-1051, :392-398).
//  2. sfa_attn_kernel -- one work-group (4 waves) per (query row, block of 64
//     heads). Per tile of 32 tokens the gathered rows [D | Dr] are staged in
//     LDS with 16-byte loads; each wave computes S = Q K^T for 16 heads with
//     v_mfma_f32_16x16x32 (Q resident in VGPRs), runs the online softmax in
//     fp32 (row max via lane shuffles, row sums kept per lane), writes P (io
//     dtype) and the rescale factors to LDS; then each wave accumulates
//     O[64 heads, D/4 columns] += P V with v_mfma_f32_32x32x16, V being the
//     same LDS rows (value = key). O never leaves VGPRs until the epilogue
//     divides by the row sum and stores the io-dtype output and LSE stats.
#include "dsa_common.hpp"

namespace dsa {
namespace {

constexpr int DR = 64;
constexpr int HB = 64;   // heads per work-group
constexpr int BN = 32;   // tokens per tile
constexpr int NWAVE = 4;

struct RowInfo {
  int b, s1, aq, ak, threshold;
  bool active;
};

__device__ __forceinline__ RowInfo row_info(const SfaArgs& a, int r) {
  RowInfo ri;
  ri.b = batch_of_row(a.row_start, a.batch, r);
  ri.s1 = r - a.row_start[ri.b];
  ri.aq = a.act_q[ri.b];
  ri.ak = a.act_k[ri.b];
  ri.active = ri.s1 < ri.aq;
  if (a.sparse_mode != 0 && ri.s1 < ri.aq - ri.ak) ri.active = false;  // numpy_golden:125-126
  ri.threshold = a.sparse_mode == 0 ? ri.ak : ri.ak - ri.aq + ri.s1 + 1;
  if (ri.threshold <= 0) ri.active = false;                             // numpy_golden:131-132
  return ri;
}

// ---------------------------------------------------------------- kernel 1
constexpr int TOK_TPB = 256;

__global__ __launch_bounds__(TOK_TPB) void sfa_tokens_kernel(SfaArgs a, int cap, int32_t* counts,
                                                             int32_t* tokens) {
  __shared__ int s_first_neg;
  __shared__ int wsum[TOK_TPB / 64];
  const int r = blockIdx.x;
  const RowInfo ri = row_info(a, r);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (!ri.active) {
    if (tid == 0) counts[r] = 0;
    return;
  }
  const int bs = a.sbs;
  const int64_t ceil_blocks = ((int64_t)ri.threshold + bs - 1) / bs;
  const int nscan0 = (int)((int64_t)a.topk < ceil_blocks ? a.topk : ceil_blocks);
  const int32_t* ids = a.sidx + (int64_t)r * a.topk;
  if (tid == 0) s_first_neg = nscan0;
  __syncthreads();
  for (int i = tid; i < nscan0; i += TOK_TPB)
    if (ids[i] == -1) atomicMin(&s_first_neg, i);
  __syncthreads();
  const int nscan = s_first_neg;
  const int end_lim = ri.ak < ri.threshold ? ri.ak : ri.threshold;
  // each thread owns a contiguous run of entries so the block scan keeps order
  const int per = (nscan + TOK_TPB - 1) / TOK_TPB;
  const int i0 = tid * per, i1 = (i0 + per < nscan ? i0 + per : nscan);
  int my = 0;
  for (int i = i0; i < i1; ++i) {
    const int id = ids[i];
    if (id < 0) continue;  // only -1 is defined (stops the scan); other negatives are skipped
    const int64_t begin = (int64_t)id * bs;
    if (begin >= ri.threshold) continue;
    const int64_t e = begin + bs < end_lim ? begin + bs : end_lim;
    if (e > begin) my += (int)(e - begin);
  }
  // block exclusive scan of `my`
  int v = my;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int n = __shfl_up(v, o);
    if (lane >= o) v += n;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < TOK_TPB / 64; ++w) {
    off += w < wave ? wsum[w] : 0;
    tot += wsum[w];
  }
  int pos = off + v - my;
  int32_t* out = tokens + (int64_t)r * cap;
  for (int i = i0; i < i1; ++i) {
    const int id = ids[i];
    if (id < 0) continue;
    const int64_t begin = (int64_t)id * bs;
    if (begin >= ri.threshold) continue;
    const int64_t e = begin + bs < end_lim ? begin + bs : end_lim;
    for (int64_t t = begin; t < e; ++t) {
      int32_t phys;
      if (a.block_table) {
        const int64_t bi = t / a.page_bs;
        const int blk = bi < a.max_blocks ? a.block_table[(int64_t)ri.b * a.max_blocks + bi] : -1;
        const int64_t p = blk < 0 ? -1 : (int64_t)blk * a.page_bs + t % a.page_bs;
        phys = (p >= 0 && p < a.key_rows) ? (int32_t)p : -1;
      } else {
        const int64_t p = (int64_t)a.key_start[ri.b] + t;
        phys = (t < a.s2 && p < a.key_rows) ? (int32_t)p : -1;
      }
      out[pos++] = phys;
    }
  }
  if (tid == 0) counts[r] = tot;
}

// ---------------------------------------------------------------- kernel 2
template <int D> struct AttnCfg {
  static constexpr int DK = D + DR;           // contraction length of Q K^T
  static constexpr int KS = DK / 32;          // 16x16x32 k-steps
  static constexpr int PITCH = DK + 8;        // LDS row pitch (elements)
  static constexpr int CH_ROW = DK / 8;       // 16-byte chunks per token row
  static constexpr int CH_TILE = BN * CH_ROW;
  static constexpr int DW = D / NWAVE;        // output columns per wave
  static constexpr int NT = DW / 32;          // 32-wide N tiles per wave
  static constexpr int PP = BN + 8;           // P tile pitch (elements)
};

template <int IO, int D>
__global__ __launch_bounds__(NWAVE * 64) void sfa_attn_kernel(SfaArgs a, int cap,
                                                              const int32_t* counts,
                                                              const int32_t* tokens) {
  using C = AttnCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t kv[BN * C::PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t pt[HB * C::PP];
  __shared__ float s_alpha[HB];
  __shared__ float s_l[HB];
  __shared__ int s_tok[BN];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.x;
  const int h0 = blockIdx.y * HB;
  const int ntok = counts[r];
  const int32_t* toks = tokens + (int64_t)r * cap;
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out);

  if (ntok == 0) {  // skipped row: zeros (out, stats)
    for (int i = threadIdx.x; i < HB * D; i += NWAVE * 64) {
      const int h = h0 + i / D;
      if (h < a.n1) out[((int64_t)r * a.n1 + h) * D + (i % D)] = 0;
    }
    if (a.sm_max && threadIdx.x < HB && h0 + (int)threadIdx.x < a.n1) {
      a.sm_max[(int64_t)r * a.n1 + h0 + threadIdx.x] = 0.f;
      a.sm_sum[(int64_t)r * a.n1 + h0 + threadIdx.x] = 0.f;
    }
    return;
  }

  // ---- Q fragments (A of S = Q K^T): 16 heads per wave, 16x16x32 layout
  const int hq = h0 + wave * 16 + (lane & 15);
  const uint16_t* qn = reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)r * a.n1 + hq) * D;
  const uint16_t* qr = reinterpret_cast<const uint16_t*>(a.qr) + ((int64_t)r * a.n1 + hq) * DR;
  uint4 qf[C::KS];
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) {
    const int e = ks * 32 + (lane >> 4) * 8;
    if (hq < a.n1)
      qf[ks] = e < D ? ldg16(qn + e) : ldg16(qr + (e - D));
    else
      qf[ks] = make_uint4(0, 0, 0, 0);
  }

  constexpr float LOG2E = 1.4426950408889634f;
  float m_run[4], l_part[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) { m_run[i] = -INFINITY; l_part[i] = 0.f; }
  f32x16 o[2][C::NT];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[mt][nt][i] = 0.f;

  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(a.k);
  const uint16_t* krbase = reinterpret_cast<const uint16_t*>(a.kr);
  const int ntiles = (ntok + BN - 1) / BN;

  for (int t = 0; t < ntiles; ++t) {
    const int tb = t * BN;
    const int nvalid = ntok - tb < BN ? ntok - tb : BN;
    if (threadIdx.x < BN) s_tok[threadIdx.x] = threadIdx.x < nvalid ? toks[tb + threadIdx.x] : -1;
    __syncthreads();
    // ---- gather the tile's rows [D | Dr] into LDS
    for (int ch = threadIdx.x; ch < C::CH_TILE; ch += NWAVE * 64) {
      const int tk = ch / C::CH_ROW, part = ch % C::CH_ROW;
      const int phys = s_tok[tk];
      uint4 v = make_uint4(0, 0, 0, 0);
      if (phys >= 0) {
        const int e = part * 8;
        v = e < D ? ldg16(kbase + (int64_t)phys * D + e) : ldg16(krbase + (int64_t)phys * DR + (e - D));
      }
      *reinterpret_cast<uint4*>(&kv[tk * C::PITCH + part * 8]) = v;
    }
    __syncthreads();

    // ---- S = Q K^T for this wave's 16 heads x 32 tokens
    f32x4 s[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      s[sub] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint16_t* bp = &kv[(sub * 16 + (lane & 15)) * C::PITCH + (lane >> 4) * 8];
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks)
        s[sub] = Mfma<IO>::m16(qf[ks], *reinterpret_cast<const uint4*>(bp + ks * 32), s[sub]);
    }
    // lane holds heads wave*16 + (lane>>4)*4 + i, tokens sub*16 + (lane&15)
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // x = score * scale in natural units, so m_run is exactly the golden's max
      const float x0 = (lane & 15) < nvalid ? s[0][i] * a.scale : -INFINITY;
      const float x1 = 16 + (lane & 15) < nvalid ? s[1][i] * a.scale : -INFINITY;
      float mx = fmaxf(x0, x1);
#pragma unroll
      for (int o2 = 1; o2 < 16; o2 <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o2));
      const float mnew = fmaxf(m_run[i], mx);  // finite: token 0 of every tile is valid
      alpha[i] = exp2f((m_run[i] - mnew) * LOG2E);
      m_run[i] = mnew;
      const float p0 = exp2f((x0 - mnew) * LOG2E), p1 = exp2f((x1 - mnew) * LOG2E);
      l_part[i] = l_part[i] * alpha[i] + p0 + p1;
      const int hl = wave * 16 + (lane >> 4) * 4 + i;
      pt[hl * C::PP + (lane & 15)] = from_f32<IO>(p0);
      pt[hl * C::PP + 16 + (lane & 15)] = from_f32<IO>(p1);
      if ((lane & 15) == 0) s_alpha[hl] = alpha[i];
    }
    __syncthreads();

    // ---- O[64 heads, this wave's D/4 columns] = alpha * O + P V
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      float al[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) al[i] = s_alpha[mt * 32 + m32_row(i, lane)];
#pragma unroll
      for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[mt][nt][i] *= al[i];
    }
#pragma unroll
    for (int kq = 0; kq < BN / 16; ++kq) {
      uint4 pa[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
        pa[mt] = *reinterpret_cast<const uint4*>(&pt[(mt * 32 + (lane & 31)) * C::PP + kq * 16 + (lane >> 5) * 8]);
#pragma unroll
      for (int nt = 0; nt < C::NT; ++nt) {
        const int dcol = wave * C::DW + nt * 32 + (lane & 31);
        const uint16_t* vp = &kv[(kq * 16 + (lane >> 5) * 8) * C::PITCH + dcol];
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          w[j] = (uint32_t)vp[(2 * j) * C::PITCH] | ((uint32_t)vp[(2 * j + 1) * C::PITCH] << 16);
        const uint4 vb = make_uint4(w[0], w[1], w[2], w[3]);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) o[mt][nt] = Mfma<IO>::m32(pa[mt], vb, o[mt][nt]);
      }
    }
    __syncthreads();
  }

  // ---- epilogue: finish row sums, normalise, store
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float l = l_part[i];
#pragma unroll
    for (int o2 = 1; o2 < 16; o2 <<= 1) l += __shfl_xor(l, o2);
    const int hl = wave * 16 + (lane >> 4) * 4 + i;
    if ((lane & 15) == 0) {
      s_l[hl] = l;
      const int h = h0 + hl;
      if (a.sm_max && h < a.n1) {
        a.sm_max[(int64_t)r * a.n1 + h] = m_run[i];
        a.sm_sum[(int64_t)r * a.n1 + h] = l;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int hl = mt * 32 + m32_row(i, lane);
      const int h = h0 + hl;
      if (h >= a.n1) continue;
      const float inv = 1.f / s_l[hl];
#pragma unroll
      for (int nt = 0; nt < C::NT; ++nt) {
        const int dcol = wave * C::DW + nt * 32 + (lane & 31);
        out[((int64_t)r * a.n1 + h) * D + dcol] = from_f32<IO>(o[mt][nt][i] * inv);
      }
    }
  }
}

template <int IO>
hipError_t launch_attn(const SfaArgs& a, hipStream_t s, int cap, const int32_t* counts,
                       const int32_t* tokens) {
  dim3 grid(a.total_rows, (a.n1 + HB - 1) / HB), block(NWAVE * 64);
  switch (a.d) {
    case 128: hipLaunchKernelGGL((sfa_attn_kernel<IO, 128>), grid, block, 0, s, a, cap, counts, tokens); break;
    case 256: hipLaunchKernelGGL((sfa_attn_kernel<IO, 256>), grid, block, 0, s, a, cap, counts, tokens); break;
    case 512: hipLaunchKernelGGL((sfa_attn_kernel<IO, 512>), grid, block, 0, s, a, cap, counts, tokens); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace
}  // namespace dsa

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t sfa_workspace_bytes(int total_rows, int n1, int d, int topk, int sbs, int kv_splits) {
  (void)n1; (void)d; (void)kv_splits;
  const size_t cap = (size_t)topk * (size_t)sbs;
  return align256((size_t)total_rows * 4) + align256((size_t)total_rows * cap * 4);
}

hipError_t launch_sfa_fwd(const SfaArgs& a, hipStream_t s) {
  if (a.total_rows <= 0) return hipSuccess;
  const int cap = a.topk * a.sbs;
  int32_t* counts = reinterpret_cast<int32_t*>(a.ws);
  int32_t* tokens = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(a.ws) + align256((size_t)a.total_rows * 4));
  hipLaunchKernelGGL(dsa::sfa_tokens_kernel, dim3(a.total_rows), dim3(dsa::TOK_TPB), 0, s, a, cap,
                     counts, tokens);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return a.io == dsa::IO_BF16 ? dsa::launch_attn<dsa::IO_BF16>(a, s, cap, counts, tokens)
                              : dsa::launch_attn<dsa::IO_F16>(a, s, cap, counts, tokens);
}
