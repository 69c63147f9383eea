// MLA absorbed (latent-cache) decode for gfx950.
//
//   O[b,h,:] = softmax_t( scale * Q[b,h,:] . KV[b,t,:] ) . KV[b,t,0:512]
//
// with Q[B,H,576], KV[B,T,576] (512 latent + 64 rope), O[B,H,512], bf16.
// This is softmax attention with one shared key/value head: the oracle is
// analysis/wave15-attention-architecture/reference/pytorch_reference_mla.py:66-81
// (`mla_naive`) with K := KV[b], V := KV[b][:, :512] broadcast to all heads,
// which is the weight-absorbed decode form of
// analysis/wave15-attention-research/MECHANISMS.md:91-94, 115-120.
//
// MI355X design (HBM-bound: the latent cache is read exactly once):
//  * A workgroup owns one sequence b, one slice of T ("split") and 64 heads;
//    its 4 waves take 16 heads each.  Each 32-token KV tile is fetched from
//    HBM once (128-bit, coalesced rows) and shared by the 64 heads in LDS.
//    When a sequence needs two head groups, they sit on the same XCD so
//    the second read of a tile hits L2.
//  * Scores are computed transposed, S^T = KV · Q^T, with 16x16x32 MFMAs:
//    lane l owns head l%16 and 4 tokens per 16-token tile, so the softmax
//    reductions are lane-local plus two permlane swaps (xor 16, xor 32).
//  * P stays in registers as the B operand of O^T = V^T · P^T; V^T is built
//    in LDS from the same KV tile (registers transposed with byte permutes
//    on the way in), so the cache is never re-read from HBM.
//  * T is split across workgroups to fill the 256 CUs; each split writes
//    (m, l, unnormalised o) to the workspace and a second kernel merges the
//    splits with the log-sum-exp rule.  With one split, O is written directly.
#include "mx_common.h"

namespace mx {
namespace mla {

constexpr int DQK = 576;
constexpr int DV = 512;
constexpr int BT = 32;                  // tokens per KV tile
constexpr int HPW = 16;                 // heads per wave
constexpr int NWAVES = 4;
constexpr int NT = 64 * NWAVES;
constexpr int HPG = HPW * NWAVES;       // heads per workgroup
constexpr int KS = DQK / 32;            // 18 k-steps of QK^T
constexpr int VT = DV / 16;             // 32 dv tiles of O^T
constexpr int ROW_B = DQK * 2;          // 1152 bytes per KV row in LDS
constexpr int K_BYTES = BT * ROW_B;     // 36864
constexpr int VT_ROW_B = BT * 2;        // 64 bytes per V^T row
constexpr int V_BYTES = DV * VT_ROW_B;  // 32768
constexpr int STAGE = K_BYTES + V_BYTES;
constexpr int LDS_TOTAL = 2 * STAGE;    // 139264
constexpr float kLog2e = 1.4426950408889634f;

// KV tile: chunk c of row r; chunks XOR-swizzled inside aligned groups of 8.
__device__ __forceinline__ int kv_off(int r, int c) { return r * ROW_B + (((c & ~7) | ((c ^ r) & 7)) << 4); }
// V^T tile: 8-byte chunk ch (4 tokens) of dv row d.
__device__ __forceinline__ int vt_off(int d, int ch) { return d * VT_ROW_B + ((ch ^ ((d >> 2) & 7)) << 3); }

struct Split {
  int nsplit;
  int tps;  // tokens per split (multiple of BT)
};

__host__ __device__ inline Split pick_split(int B, int H, int T) {
  const int hg = (H + HPG - 1) / HPG;
  const int nblk = (T + BT - 1) / BT;
  // Aim for >= 256 workgroups (one per CU) without splits shorter than
  // 4 tiles; never more splits than tiles.
  int ns = 1;
  while ((long long)B * hg * ns < 256 && ns * 2 <= nblk / 4) ns *= 2;
  const int blocks_per = (nblk + ns - 1) / ns;
  Split s;
  s.nsplit = (nblk + blocks_per - 1) / blocks_per;
  s.tps = blocks_per * BT;
  return s;
}

__global__ __launch_bounds__(NT, 1) void mla_decode_kernel(const uint16_t* __restrict__ Q,
                                                          const uint16_t* __restrict__ KV,
                                                          uint16_t* __restrict__ O, float* __restrict__ ws_o,
                                                          float* __restrict__ ws_ml, int B, int H, int T,
                                                          float sl2, int nsplit, int tps) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4;   // lane group (4 groups of 16)
  const int hl = lane & 15;  // head within the wave

  const int HG = (H + HPG - 1) / HPG;
  const int nwg = B * HG * nsplit;
  const int id = xcd_remap(blockIdx.x, nwg);
  const int hg = id % HG;
  const int s = (id / HG) % nsplit;
  const int b = id / (HG * nsplit);

  const int head = hg * HPG + wave * HPW + hl;
  const bool head_ok = head < H;
  const int t0 = s * tps;
  const int t1 = min(T, t0 + tps);
  const int nblk = (t1 - t0 + BT - 1) / BT;

  // Q^T fragments: lane holds head `head`, d = 32 ks + 8 g .. +7.
  u32x4 qf[KS];
  const uint16_t* qrow = Q + ((size_t)b * H + (head_ok ? head : 0)) * DQK;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = head_ok ? ld128(qrow + ks * 32 + g * 8) : u32x4{0, 0, 0, 0};

  const uint16_t* kvb = KV + (size_t)b * T * DQK;

  // Staging: latent part as two 4(tok) x 8(dv) blocks per thread, rope part
  // as one 16-byte chunk per thread.
  const int v_dvb = tid & 63;       // dv block (8 columns)
  const int v_tb = tid >> 6;        // token block 0..3 (and +4)
  const int r_row = tid >> 3;       // rope row 0..31
  const int r_chunk = 64 + (tid & 7);
  u32x4 rv[2][4], rr;

  auto load_tile = [&](int tok0) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = tok0 + (v_tb + 4 * i) * 4 + r;
        rv[i][r] = (tok < t1) ? ld128(kvb + (size_t)tok * DQK + v_dvb * 8) : u32x4{0, 0, 0, 0};
      }
    const int tok = tok0 + r_row;
    rr = (tok < t1) ? ld128(kvb + (size_t)tok * DQK + r_chunk * 8) : u32x4{0, 0, 0, 0};
  };
  auto store_tile = [&](int stage) {
    unsigned char* sk = smem + stage * STAGE;
    unsigned char* sv = sk + K_BYTES;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int tb = v_tb + 4 * i;
#pragma unroll
      for (int r = 0; r < 4; ++r) *reinterpret_cast<u32x4*>(sk + kv_off(tb * 4 + r, v_dvb)) = rv[i][r];
      u32x2 cols[8];
      transpose4x8_b16(rv[i], cols);
#pragma unroll
      for (int c = 0; c < 8; ++c) *reinterpret_cast<u32x2*>(sv + vt_off(v_dvb * 8 + c, tb)) = cols[c];
    }
    *reinterpret_cast<u32x4*>(sk + kv_off(r_row, r_chunk)) = rr;
  };

  f32x4 acc[VT];
#pragma unroll
  for (int i = 0; i < VT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_run = 0.f;

  if (nblk > 0) {
    load_tile(t0);
    store_tile(0);
  }
  __syncthreads();

  for (int blk = 0; blk < nblk; ++blk) {
    const int cur = blk & 1;
    const int tok0 = t0 + blk * BT;
    if (blk + 1 < nblk) load_tile(tok0 + BT);
    const unsigned char* sk = smem + cur * STAGE;
    const unsigned char* sv = sk + K_BYTES;

    // S^T: two 16-token tiles x 16 heads, contraction over 576.
    f32x4 sc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      sc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(sk + kv_off(tt * 16 + hl, ks * 4 + g));
        sc[tt] = mfma16<BF16>(kf, qf[ks], sc[tt]);
      }
    }
    // lane holds tokens tok0 + 16 tt + 4 g + j
    const bool need_mask = tok0 + BT > t1;
    float mx = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x = sc[tt][j] * sl2;
        if (need_mask && tok0 + 16 * tt + 4 * g + j >= t1) x = -INFINITY;
        sc[tt][j] = x;
        mx = fmaxf(mx, x);
      }
    mx = max_xor16(mx);
    mx = max_xor32(mx);
    const float m_new = fmaxf(m_run, mx);
    const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float lsum = 0.f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p = __builtin_amdgcn_exp2f(sc[tt][j] - m_new);
        sc[tt][j] = p;
        lsum += p;
      }
    l_run = l_run * corr + lsum;
    const u32x4 pf{pack_bf16x2(sc[0][0], sc[0][1]), pack_bf16x2(sc[0][2], sc[0][3]), pack_bf16x2(sc[1][0], sc[1][1]),
                   pack_bf16x2(sc[1][2], sc[1][3])};
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      const int d = vt * 16 + hl;
      const u32x2 lo = *reinterpret_cast<const u32x2*>(sv + vt_off(d, g));
      const u32x2 hi = *reinterpret_cast<const u32x2*>(sv + vt_off(d, 4 + g));
      acc[vt] = mfma16<BF16>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pf, acc[vt] * corr);
    }

    if (blk + 1 < nblk) store_tile(cur ^ 1);
    __syncthreads();
  }

  // lane holds head `head`, dv = 16 vt + 4 g + j
  float l_tot = sum_xor16(l_run);
  l_tot = sum_xor32(l_tot);
  if (!head_ok) return;
  if (nsplit == 1) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint16_t* orow = O + ((size_t)b * H + head) * DV;
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
      st64(orow + vt * 16 + 4 * g,
           u32x2{pack_bf16x2(acc[vt][0] * inv, acc[vt][1] * inv), pack_bf16x2(acc[vt][2] * inv, acc[vt][3] * inv)});
    return;
  }
  const size_t pidx = ((size_t)b * nsplit + s) * H + head;
  float* po = ws_o + pidx * DV;
#pragma unroll
  for (int vt = 0; vt < VT; ++vt) *reinterpret_cast<f32x4*>(po + vt * 16 + 4 * g) = acc[vt];
  if (g == 0) {
    ws_ml[2 * pidx] = m_run;
    ws_ml[2 * pidx + 1] = l_tot;
  }
}

// Merge the per-split softmax states:  o = sum_s w_s o_s / sum_s w_s l_s,
// w_s = 2^(m_s - max_s m_s).  One workgroup per (b, h), 128 threads x 4 dv.
__global__ __launch_bounds__(128) void mla_combine_kernel(const float* __restrict__ ws_o,
                                                         const float* __restrict__ ws_ml,
                                                         uint16_t* __restrict__ O, int H, int nsplit) {
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh % H;
  const int d = threadIdx.x * 4;
  float mmax = -1e30f;
  for (int s = 0; s < nsplit; ++s) mmax = fmaxf(mmax, ws_ml[2 * (((size_t)b * nsplit + s) * H + h)]);
  f32x4 o{0.f, 0.f, 0.f, 0.f};
  float l = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const size_t pidx = ((size_t)b * nsplit + s) * H + h;
    const float w = __builtin_amdgcn_exp2f(ws_ml[2 * pidx] - mmax);
    l = fmaf(w, ws_ml[2 * pidx + 1], l);
    o += w * *reinterpret_cast<const f32x4*>(ws_o + pidx * DV + d);
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  st64(O + (size_t)bh * DV + d, u32x2{pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv)});
}

inline size_t workspace_bytes(int B, int H, int T) {
  const Split sp = pick_split(B, H, T);
  if (sp.nsplit <= 1) return 0;
  return (size_t)B * sp.nsplit * H * (DV + 2) * sizeof(float);
}

}  // namespace mla
}  // namespace mx

extern "C" size_t mx_mla_decode_workspace(int B, int H, int T, int d_latent) {
  if (B <= 0 || H <= 0 || T <= 0 || d_latent != mx::mla::DV) return 0;
  return mx::mla::workspace_bytes(B, H, T);
}

extern "C" int mx_mla_decode(const void* Q, const void* KV, void* O, int B, int H, int T, int d_latent, int d_rope,
                             float scale, void* workspace, size_t ws_bytes, void* stream) {
  using namespace mx::mla;
  if (!Q || !KV || !O) return MX_ERR_NULL;
  if (B <= 0 || H <= 0 || T <= 0) return MX_ERR_SHAPE;
  if (d_latent != DV || d_rope != DQK - DV) return MX_ERR_UNSUPPORTED;
  if (!(scale > 0.f) || !__builtin_isfinite(scale)) return MX_ERR_SHAPE;
  if ((long long)B * T * DQK > (1LL << 40) || (long long)B * H > (1LL << 30)) return MX_ERR_SHAPE;
  if (((uintptr_t)Q | (uintptr_t)KV | (uintptr_t)O) & 15) return MX_ERR_ALIGN;
  const Split sp = pick_split(B, H, T);
  const size_t need = workspace_bytes(B, H, T);
  if (need > 0 && (!workspace || ws_bytes < need)) return MX_ERR_WORKSPACE;
  if (need > 0 && ((uintptr_t)workspace & 15)) return MX_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const int HG = (H + HPG - 1) / HPG;
  const long long grid = (long long)B * HG * sp.nsplit;
  if (grid > 0x7fffffffLL) return MX_ERR_SHAPE;
  float* ws_o = (float*)workspace;
  float* ws_ml = need ? ws_o + (size_t)B * sp.nsplit * H * DV : nullptr;
  MX_RETURN_IF_HIP(
      hipFuncSetAttribute((const void*)mla_decode_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_TOTAL));
  hipLaunchKernelGGL(mla_decode_kernel, dim3((unsigned)grid), dim3(NT), LDS_TOTAL, s, (const uint16_t*)Q,
                     (const uint16_t*)KV, (uint16_t*)O, ws_o, ws_ml, B, H, T, scale * kLog2e, sp.nsplit, sp.tps);
  MX_RETURN_IF_HIP(hipGetLastError());
  if (sp.nsplit > 1) {
    hipLaunchKernelGGL(mla_combine_kernel, dim3(B * H), dim3(DV / 4), 0, s, ws_o, ws_ml, (uint16_t*)O, H, sp.nsplit);
    MX_RETURN_IF_HIP(hipGetLastError());
  }
  return MX_OK;
}
