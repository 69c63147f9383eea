// Gated-DeltaNet (GDN) and Kimi-Delta-Attention (KDA) single-token decode
// for gfx950.
//
// Math (per batch b, value head hv, key head hk = hv / (Hv/Hk)), following
// analysis/wave15-attention-architecture/reference/pytorch_reference_gdn.py:38-91
// and cutile-attn-gdn/main.py:92-185:
//     u      = k^T (alpha S)                 (d_v)
//     r      = v - u
//     S'     = alpha S + beta k r^T          (d_k x d_v, fp32)
//     o      = S'^T q
// The output is formed without a second pass over S' through
//     o = alpha (q^T S) + beta (q.k) r,
// so both reductions (k^T S and q^T S) come out of the single read of S.
//
// KDA (cutile-attn-kda/main.py:187-271, oracle
// analysis/wave15-attention-architecture/reference/pytorch_reference_kda.py:42-73)
// replaces the scalar alpha by a per-row decay e = exp(g) (d_k values):
//     u = (e*k)^T S,  r = v - u,  S' = diag(e) S + beta k r^T,
//     o = (e*q)^T S + beta (q.k) r
// — the same single-pass kernel with e folded into the row coefficients.
//
// Layout and schedule (bandwidth-bound: 2 x d_k x d_v x 4 bytes per head):
//  * one workgroup per (b, hv, column block of BV values of d_v) — every
//    column of S is independent, so the d_v split needs no cross-workgroup
//    reduction (the reference tiles d_v the same way, main.py:228-246).  BV
//    is chosen at launch so that small batches still spread over the CUs;
//  * NT = d_k*BV/64 threads (<= 1024) so every thread keeps exactly 16 rows x 4
//    columns (64 fp32) of the state in VGPRs between the read and the
//    write — S is read once and written once, with 128-bit loads and
//    non-temporal stores, BV/4 threads covering a row segment;
//  * the BV-wide partial reductions over each thread's 16 rows meet in LDS
//    (d_k/16 row groups), one barrier, then every thread forms u, r, o for
//    its own columns and streams its rows of S' back out.
#include "mx_common.h"

namespace mx {
namespace gdn {

// Gate inputs of one launch.  GDN: scalar decay alpha and beta per (b, hv),
// fp32.  KDA: per-channel log-gate g[b, h, 0..d_k) and beta[b, h] in the
// 16-bit I/O type, decay exp(g).
struct Gates {
  const float* alpha;      // GDN
  const float* beta;       // GDN
  const uint16_t* g;       // KDA
  const uint16_t* beta16;  // KDA
};

template <int DK, int BV, typename T, bool KDA>
__global__ __launch_bounds__(DK * BV / 64) void gdn_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, Gates gt,
    const float* S_in, float* S_out, uint16_t* __restrict__ o, int Hk, int Hv, int DV) {
  constexpr int NT = DK * BV / 64;
  constexpr int TC = BV / 4;   // threads across a row segment
  constexpr int RG = NT / TC;  // row groups (= DK / 16)
  constexpr int RPT = DK / RG; // rows per thread (= 16)
  static_assert(RPT == 16, "16 rows per thread");

  __shared__ float qs[DK], ks[DK], es[KDA ? DK : 1];
  __shared__ __align__(16) float red_u[RG][BV];
  __shared__ __align__(16) float red_w[RG][BV];
  __shared__ float red_qk[RG];

  const int nvb = DV / BV;
  const int bh = blockIdx.x / nvb;  // b * Hv + hv
  const int vblk = blockIdx.x % nvb;
  const int b = bh / Hv, hv = bh % Hv;
  const int hk = hv / (Hv / Hk);
  const int t = threadIdx.x;
  const int cg = t % TC, rg = t / TC;
  const int cl = cg * 4;              // column within the block
  const int c0 = vblk * BV + cl;      // column within d_v

  const size_t sbase = (size_t)bh * DK * DV;
  const float* Sin = S_in + sbase;
  float* Sout = S_out + sbase;

  // Issue the 16 state loads first: they dominate and need to be in flight.
  // Ordinary loads: on MI355X the non-temporal form streams slower (a
  // 134 MB copy runs at ~6.9 TB/s with ordinary 128-bit loads and stores,
  // ~5.5-6.2 TB/s with non-temporal ones); the stores stay non-temporal,
  // which measured fastest for this kernel.
  f32x4 s[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + RG * r;
    s[r] = __builtin_bit_cast(f32x4, ld128(Sin + (size_t)i * DV + c0));
  }

  const size_t qkbase = ((size_t)b * Hk + hk) * DK;
  for (int i = t; i < DK; i += NT) {
    qs[i] = T::to_f32(q[qkbase + i]);
    ks[i] = T::to_f32(k[qkbase + i]);
    if constexpr (KDA) es[i] = expf(T::to_f32(gt.g[(size_t)bh * DK + i]));
  }
  const size_t vbase = (size_t)bh * DV + c0;
  const u32x2 vv = ld64(v + vbase);
  const float vf[4] = {T::to_f32(vv[0] & 0xffffu), T::to_f32(vv[0] >> 16), T::to_f32(vv[1] & 0xffffu),
                       T::to_f32(vv[1] >> 16)};
  // GDN: the scalar decay multiplies the reductions once at the end (a);
  // KDA: each row's decay e_i is folded into that row's coefficients.
  const float a = KDA ? 1.f : gt.alpha[bh];
  const float be = KDA ? T::to_f32(gt.beta16[bh]) : gt.beta[bh];
  __syncthreads();

  float u[4] = {0.f, 0.f, 0.f, 0.f}, w[4] = {0.f, 0.f, 0.f, 0.f};
  float qk = 0.f;
  float kr[RPT], er[KDA ? RPT : 1];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + RG * r;
    float ki = ks[i], qi = qs[i];
    kr[r] = ki;
    qk = fmaf(qi, ki, qk);
    if constexpr (KDA) {
      er[r] = es[i];
      ki *= er[r];
      qi *= er[r];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u[c] = fmaf(ki, s[r][c], u[c]);
      w[c] = fmaf(qi, s[r][c], w[c]);
    }
  }
  *reinterpret_cast<f32x4*>(&red_u[rg][cl]) = f32x4{u[0], u[1], u[2], u[3]};
  *reinterpret_cast<f32x4*>(&red_w[rg][cl]) = f32x4{w[0], w[1], w[2], w[3]};
  if (cg == 0) red_qk[rg] = qk;
  __syncthreads();

  f32x4 ut{0.f, 0.f, 0.f, 0.f}, wt{0.f, 0.f, 0.f, 0.f};
  float qkt = 0.f;
#pragma unroll
  for (int gi = 0; gi < RG; ++gi) {
    ut += *reinterpret_cast<const f32x4*>(&red_u[gi][cl]);
    wt += *reinterpret_cast<const f32x4*>(&red_w[gi][cl]);
    qkt += red_qk[gi];
  }

  float res[4], of[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    res[c] = vf[c] - a * ut[c];                  // r = v - alpha k^T S
    of[c] = fmaf(be * qkt, res[c], a * wt[c]);   // o = alpha q^T S + beta (q.k) r
  }

#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + RG * r;
    const float bk = be * kr[r];
    const float ar = KDA ? er[r] : a;
    f32x4 nv;
#pragma unroll
    for (int c = 0; c < 4; ++c) nv[c] = fmaf(bk, res[c], ar * s[r][c]);
    st128_nt(Sout + (size_t)i * DV + c0, __builtin_bit_cast(u32x4, nv));
  }
  if (rg == 0) {
    st64(o + vbase, u32x2{T::pack2(of[0], of[1]), T::pack2(of[2], of[3])});
  }
}

template <int DK, int BV, typename T, bool KDA>
static int launch(const void* q, const void* k, const void* v, const Gates& gt, const float* S_in, float* S_out,
                  void* o, int B, int Hk, int Hv, int dv, hipStream_t s) {
  const long long grid = (long long)B * Hv * (dv / BV);
  if (grid > 0x7fffffffLL) return MX_ERR_SHAPE;
  hipLaunchKernelGGL((gdn_decode_kernel<DK, BV, T, KDA>), dim3((unsigned)grid), dim3(DK * BV / 64), 0, s,
                     (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, gt, S_in, S_out, (uint16_t*)o, Hk,
                     Hv, dv);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}

// Column-block width.  At most 65536/d_k columns, so a workgroup of
// d_k*BV/64 threads stays within 1024 (d_k = 512: BV <= 128).  Start from
// that and halve while the grid has fewer
// than 4096 workgroups (16 per CU: small workgroups keep the last wave of
// the grid short) but not below 64 columns (256-byte row segments stream
// well; 64-byte ones do not: 4.0 vs 6.5 TB/s at B4 H64 d256).  Only when
// that still leaves fewer than 1024 workgroups, keep halving down to the
// narrowest allowed width (>= 16 and >= 4096/d_k, i.e. one wave per
// workgroup) for parallelism.  Measured choices: B64 Hv32 d128 -> 64
// (4096 workgroups, ~7% faster than 128), B4 H64 d256 -> 64, B1 H16 d256
// -> 16.
static int pick_bv(int B, int Hv, int dk, int dv) {
  const int min_bv = (4096 / dk > 16) ? 4096 / dk : 16;
  auto groups = [&](int bv) { return (long long)B * Hv * (dv / bv); };
  int bv = dv < 65536 / dk ? dv : 65536 / dk;
  while (bv / 2 >= 64 && bv / 2 >= min_bv && groups(bv) < 4096) bv /= 2;
  while (bv / 2 >= min_bv && groups(bv) < 1024) bv /= 2;
  return bv;
}

template <int DK, typename T, bool KDA>
static int dispatch_dk(const void* q, const void* k, const void* v, const Gates& gt, const float* S_in, float* S_out,
                       void* o, int B, int Hk, int Hv, int dv, hipStream_t s) {
  const int bv = pick_bv(B, Hv, DK, dv);
#define MX_GDN_BV(BV_)                                                                                     \
  if (bv == BV_) {                                                                                         \
    if constexpr (DK * BV_ >= 4096 && DK * BV_ <= 65536)                                                   \
      return launch<DK, BV_, T, KDA>(q, k, v, gt, S_in, S_out, o, B, Hk, Hv, dv, s);                        \
  }
  MX_GDN_BV(16)
  MX_GDN_BV(32)
  MX_GDN_BV(64)
  MX_GDN_BV(128)
  MX_GDN_BV(256)
#undef MX_GDN_BV
  return MX_ERR_UNSUPPORTED;
}

template <typename T, bool KDA>
static int dispatch(const void* q, const void* k, const void* v, const Gates& gt, const float* S_in, float* S_out,
                    void* o, int B, int Hk, int Hv, int dk, int dv, hipStream_t s) {
  if (dk == 64) return dispatch_dk<64, T, KDA>(q, k, v, gt, S_in, S_out, o, B, Hk, Hv, dv, s);
  if (dk == 128) return dispatch_dk<128, T, KDA>(q, k, v, gt, S_in, S_out, o, B, Hk, Hv, dv, s);
  if (dk == 256) return dispatch_dk<256, T, KDA>(q, k, v, gt, S_in, S_out, o, B, Hk, Hv, dv, s);
  if (dk == 512) return dispatch_dk<512, T, KDA>(q, k, v, gt, S_in, S_out, o, B, Hk, Hv, dv, s);
  return MX_ERR_UNSUPPORTED;
}

// Argument checks shared by both entry points.
static int check_state(const float* S_in, const float* S_out, const void* v, const void* o, int B, int Hv, int dk,
                       int dv) {
  if (((uintptr_t)S_in | (uintptr_t)S_out) & 15) return MX_ERR_ALIGN;
  if (((uintptr_t)v | (uintptr_t)o) & 7) return MX_ERR_ALIGN;
  // The state may be updated in place; any other overlap would let one
  // workgroup overwrite rows another has not read yet.
  const size_t sbytes = (size_t)B * Hv * dk * dv * sizeof(float);
  const char* si = (const char*)S_in;
  const char* so = (const char*)S_out;
  if (si != so && si < so + sbytes && so < si + sbytes) return MX_ERR_ALIAS;
  return MX_OK;
}

}  // namespace gdn
}  // namespace mx

static bool mx_is_dim(int d) { return d == 64 || d == 128 || d == 256 || d == 512; }

extern "C" int mx_gdn_decode_block_v(int B, int Hv, int dk, int dv) {
  if (B <= 0 || Hv <= 0 || !mx_is_dim(dk) || !mx_is_dim(dv)) return 0;
  return mx::gdn::pick_bv(B, Hv, dk, dv);
}

extern "C" int mx_gdn_decode(const void* q, const void* k, const void* v, const float* alpha, const float* beta,
                             const float* S_in, float* S_out, void* o, int B, int Hk, int Hv, int dk, int dv,
                             int dtype, void* stream) {
  if (!q || !k || !v || !alpha || !beta || !S_in || !S_out || !o) return MX_ERR_NULL;
  if (B <= 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return MX_ERR_SHAPE;
  if (!mx_is_dim(dk) || !mx_is_dim(dv)) return MX_ERR_SHAPE;
  if ((long long)B * Hv > 0x7fffffffLL / 16) return MX_ERR_SHAPE;
  if (dtype != MX_DTYPE_BF16 && dtype != MX_DTYPE_F16) return MX_ERR_DTYPE;
  if (const int e = mx::gdn::check_state(S_in, S_out, v, o, B, Hv, dk, dv)) return e;
  hipStream_t s = (hipStream_t)stream;
  const mx::gdn::Gates gt{alpha, beta, nullptr, nullptr};
  if (dtype == MX_DTYPE_BF16)
    return mx::gdn::dispatch<mx::BF16, false>(q, k, v, gt, S_in, S_out, o, B, Hk, Hv, dk, dv, s);
  return mx::gdn::dispatch<mx::F16, false>(q, k, v, gt, S_in, S_out, o, B, Hk, Hv, dk, dv, s);
}

extern "C" int mx_kda_decode(const void* q, const void* k, const void* v, const void* g, const void* beta,
                             const float* S_in, float* S_out, void* o, int B, int H, int dk, int dv, int dtype,
                             void* stream) {
  if (!q || !k || !v || !g || !beta || !S_in || !S_out || !o) return MX_ERR_NULL;
  if (B <= 0 || H <= 0) return MX_ERR_SHAPE;
  if (!mx_is_dim(dk) || !mx_is_dim(dv)) return MX_ERR_SHAPE;
  if ((long long)B * H > 0x7fffffffLL / 16) return MX_ERR_SHAPE;
  if (dtype != MX_DTYPE_BF16 && dtype != MX_DTYPE_F16) return MX_ERR_DTYPE;
  if (const int e = mx::gdn::check_state(S_in, S_out, v, o, B, H, dk, dv)) return e;
  hipStream_t s = (hipStream_t)stream;
  const mx::gdn::Gates gt{nullptr, nullptr, (const uint16_t*)g, (const uint16_t*)beta};
  if (dtype == MX_DTYPE_BF16)
    return mx::gdn::dispatch<mx::BF16, true>(q, k, v, gt, S_in, S_out, o, B, H, H, dk, dv, s);
  return mx::gdn::dispatch<mx::F16, true>(q, k, v, gt, S_in, S_out, o, B, H, H, dk, dv, s);
}
