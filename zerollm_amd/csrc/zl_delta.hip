// Gated DeltaNet layer step over the B tokens of a pass (src/model/forward-qwen35.js:45-61, per-token arithmetic of
// src/compute/ref-deltanet.js:42-106), one workgroup per value head, tokens in order:
//   conv   depthwise causal conv + SiLU of the head's 3 x D channels (q and k of key head hv % nK, v of hv itself):
//          f64 dot over the window [oldest .. newest, x], stored f32; the window advances token by token;
//   l2     q normalised and scaled by 1/sqrt(D), k normalised, per token;
//   delta  S <- exp(g) S; d = beta (v - S^T k); S <- S + k d^T; o = S^T q, with the reference's f64 arithmetic and f32
//          stores; each row of S is held by 4 lanes (D/4 values each, f64 partial sums joined in a fixed order);
//   norm   gated RMSNorm of o (weights normW, gate silu(z)), then quantizeAct for the ssm_out projection.
// The head's S (D x D f32) stays in registers across the B tokens: it is read and written once per pass.
#include "zl_kernels.h"

namespace zl {

template <int D, int CK>
__global__ __launch_bounds__(4 * D) void k_deltanet(const DeltaArgs a) {
  constexpr int NT = 4 * D, NW = NT / 64, PER = D / 4;
  constexpr int ROW = D + 16;  // LDS row of q or k: the four row parts padded apart by 4 floats (distinct banks)
  constexpr int M = CK - 1;    // window length
  __shared__ float cq[DELTA_MAX_B * ROW], ck[DELTA_MAX_B * ROW], cv[DELTA_MAX_B * D], core[DELTA_MAX_B * D];
  __shared__ double gexp[DELTA_MAX_B], bet[DELTA_MAX_B];
  const int hv = blockIdx.x, kh = hv % a.nK, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = a.B;
  auto pidx = [](int i) { return i + (i / PER) * 4; };

  // ---- conv + SiLU (convStep, src/compute/ref-deltanet.js:42-55)
  const int keyDim = a.nK * D;
  if (tid < 3 * D) {
    const int grp = tid / D, i = tid - grp * D;
    const int ch = grp == 0 ? kh * D + i : grp == 1 ? keyDim + kh * D + i : 2 * keyDim + hv * D + i;
    float *win = a.conv + (((long)hv * 3 + grp) * D + i) * M;
    float w[CK], st[M > 0 ? M : 1];
    #pragma unroll
    for (int t = 0; t < CK; t++) w[t] = a.convW[(long)ch * CK + t];
    #pragma unroll
    for (int t = 0; t < M; t++) st[t] = win[t];
    for (int b = 0; b < B; b++) {
      const float cur = a.qkv[(long)b * a.ldqkv + ch];
      double acc = 0.0;
      #pragma unroll
      for (int t = 0; t < M; t++) acc += (double)w[t] * (double)st[t];
      acc += (double)w[M] * (double)cur;
      #pragma unroll
      for (int t = 0; t + 1 < M; t++) st[t] = st[t + 1];
      if (M > 0) st[M - 1] = cur;
      if (a.capConv) {  // the window after token b
        float *cw = a.capConv + (long)b * a.capStride + (((long)hv * 3 + grp) * D + i) * M;
        #pragma unroll
        for (int t = 0; t < M; t++) cw[t] = st[t];
      }
      const float y = (float)(acc / (1.0 + exp(-acc)));
      if (grp == 0) cq[b * ROW + pidx(i)] = y;
      else if (grp == 1) ck[b * ROW + pidx(i)] = y;
      else cv[b * D + i] = y;
    }
    #pragma unroll
    for (int t = 0; t < M; t++) win[t] = st[t];
  }
  // decay and write strength per token (src/model/forward-qwen35.js:55-56): beta = sigmoid(b),
  // exp(softplus(alpha + dt_bias) * ssm_a)
  if (tid < B) {
    bet[tid] = 1.0 / (1.0 + exp(-(double)a.beta[(long)tid * a.ldab + hv]));
    const double x = (double)a.alpha[(long)tid * a.ldab + hv] + (double)a.dtBias[hv];
    const double sp = x > 20.0 ? x : log1p(exp(x));
    gexp[tid] = exp(sp * (double)a.ssmA[hv]);
  }
  __syncthreads();

  // ---- L2 norms (l2normHeads, src/compute/ref-deltanet.js:61-69): one wave per (token, q or k) row
  for (int r = wave; r < 2 * B; r += NW) {
    float *row = ((r & 1) ? ck : cq) + (r >> 1) * ROW;
    double ss = 0.0;
    for (int i = lane; i < D; i += 64) { const double x = (double)row[pidx(i)]; ss += x * x; }
    ss = wave_sum_xor(ss, 64);
    const double s = ((r & 1) ? 1.0 : 1.0 / sqrt((double)D)) / sqrt(ss + a.eps);
    for (int i = lane; i < D; i += 64) row[pidx(i)] = (float)((double)row[pidx(i)] * s);
  }
  __syncthreads();

  // ---- delta rule (deltaRuleHead, src/compute/ref-deltanet.js:86-96): lane (j, p) holds S[j][p*PER .. p*PER+PER)
  const int j = tid >> 2, p = tid & 3;
  float S[PER];
  float *srow = a.ssm + ((long)hv * D + j) * D + p * PER;
  #pragma unroll
  for (int c = 0; c < PER; c += 4) {
    const float4 v4 = *(const float4 *)(srow + c);
    S[c] = v4.x; S[c + 1] = v4.y; S[c + 2] = v4.z; S[c + 3] = v4.w;
  }
  for (int b = 0; b < B; b++) {
    const double g = gexp[b], be = bet[b];
    const float *kp = ck + b * ROW + p * (PER + 4), *qp = cq + b * ROW + p * (PER + 4);
    double sk = 0.0;
    #pragma unroll
    for (int c = 0; c < PER; c++) { const double s = (double)S[c] * g; S[c] = (float)s; sk += s * (double)kp[c]; }
    sk += __shfl_xor(sk, 1);  // (p0 + p1) + (p2 + p3) on all four lanes of the row
    sk += __shfl_xor(sk, 2);
    const double d = ((double)cv[b * D + j] - sk) * be;
    double o = 0.0;
    #pragma unroll
    for (int c = 0; c < PER; c++) { const double s = (double)S[c] + (double)kp[c] * d; S[c] = (float)s; o += s * (double)qp[c]; }
    o += __shfl_xor(o, 1);
    o += __shfl_xor(o, 2);
    if (p == 0) core[b * D + j] = (float)o;
    if (a.capSsm) {  // the state after token b
      float *cs = a.capSsm + (long)b * a.capStride + ((long)hv * D + j) * D + p * PER;
      #pragma unroll
      for (int c = 0; c < PER; c += 4) *(float4 *)(cs + c) = make_float4(S[c], S[c + 1], S[c + 2], S[c + 3]);
    }
  }
  #pragma unroll
  for (int c = 0; c < PER; c += 4) *(float4 *)(srow + c) = make_float4(S[c], S[c + 1], S[c + 2], S[c + 3]);
  __syncthreads();

  // ---- gated RMSNorm (gatedRmsNormHead, src/compute/ref-deltanet.js:102-106) + quantisation, one wave per token
  for (int b = wave; b < B; b += NW) {
    const float *o = core + b * D;
    double ss = 0.0;
    for (int i = lane; i < D; i += 64) { const double x = (double)o[i]; ss += x * x; }
    ss = wave_sum_xor(ss, 64);
    const double s = 1.0 / sqrt(ss / (double)D + a.eps);
    for (int i0 = 0; i0 < D; i0 += 64) {
      const int i = i0 + lane;
      if (i < D) {  // D = 32: lanes 32-63 idle, a whole 32-lane block group
        const double zz = (double)a.z[(long)b * a.ldz + hv * D + i];
        const float v = (float)((double)o[i] * s * (double)a.normW[i] * (zz / (1.0 + exp(-zz))));
        const int col = hv * D + i;
        if (a.out) a.out[(long)b * a.ldo + col] = v;
        quant_block32(v, col, a.act, b);
      }
    }
  }
}

void launch_deltanet(const DeltaArgs &a0, int D, hipStream_t st) {
  ZL_REQUIRE(a0.K == 4, ZL_ERR_UNSUPPORTED, "Gated DeltaNet: conv kernel must be 4");
  ZL_REQUIRE(D == 32 || D == 64 || D == 128, ZL_ERR_UNSUPPORTED, "Gated DeltaNet: head size must be 32, 64 or 128");
  ZL_REQUIRE(a0.nK >= 1 && a0.nV >= 1 && a0.nV % a0.nK == 0, ZL_ERR_ARG, "Gated DeltaNet: value heads must be a multiple of key heads");
  ZL_REQUIRE(a0.act.ld >= a0.nV * D && a0.act.ld % 64 == 0, ZL_ERR_ARG, "Gated DeltaNet: activation rows too short");
  ZL_REQUIRE(!a0.capConv || a0.B <= DELTA_MAX_B, ZL_ERR_ARG, "Gated DeltaNet: capture holds one launch of tokens");
  for (int t0 = 0; t0 < a0.B; t0 += DELTA_MAX_B) {
    DeltaArgs a = a0;
    a.B = std::min(DELTA_MAX_B, a0.B - t0);
    a.qkv += (long)t0 * a.ldqkv;
    a.z += (long)t0 * a.ldz;
    a.alpha += (long)t0 * a.ldab;
    a.beta += (long)t0 * a.ldab;
    a.act = act_rows(a0.act, t0);
    if (a.out) a.out += (long)t0 * a.ldo;
    if (D == 128) hipLaunchKernelGGL((k_deltanet<128, 4>), dim3(a.nV), dim3(512), 0, st, a);
    else if (D == 64) hipLaunchKernelGGL((k_deltanet<64, 4>), dim3(a.nV), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_deltanet<32, 4>), dim3(a.nV), dim3(128), 0, st, a);
    ZL_HIP(hipGetLastError());
  }
}

}  // namespace zl
