// Gated DeltaNet layer step over the B tokens of a pass (src/model/forward-qwen35.js:45-61, per-token arithmetic of
// src/compute/ref-deltanet.js:42-106), tokens in order, DELTA_ROWS value rows (of the D) of one value head per
// workgroup:
//   conv   depthwise causal conv + SiLU of the head's q and k (key head hv % nK) and of the workgroup's v channels: f64
//          dot over the window [oldest .. newest, x], stored f32; the window advances token by token;
//   l2     q normalised and scaled by 1/sqrt(D), k normalised, per token;
//   delta  S <- exp(g) S; d = beta (v - S^T k); S <- S + k d^T; o = S^T q, with the reference's f64 arithmetic and f32
//          stores; each row of S is held by 8 lanes (D/8 values each, f64 partial sums joined in a fixed order);
//   norm   gated RMSNorm of o (weights normW, gate silu(z)), then quantizeAct for the ssm_out projection.
// Row j of the delta rule reads only S[j][.], v_j and the head's q and k, so the rows split over workgroups without any
// change of arithmetic: every workgroup convolves and normalises the head's q and k itself (the same bits in each), and
// holds its rows of S in registers across the B tokens (read and written once per pass, captured per token when asked).
// The gated norm needs the head's whole output row, so it runs as a second launch (k_delta_norm, one workgroup per value
// head) that reads the rows k_deltanet stored, and writes back the head's q and k conv windows, which every workgroup of
// the first launch read. Two launches order this without any exchange among workgroups: a hand-off by an agent-scope
// release/acquire counter inside one launch (the last workgroup of a head to arrive running the norm) measured ~6 us
// more per launch than the kernel boundary.
#include "zl_kernels.h"

namespace zl {

constexpr int DELTA_ROWS = 32;  // value rows of a head per workgroup
constexpr int DELTA_LPR = 8;    // lanes per row (DELTA_ROWS x DELTA_LPR = 256 threads)

template <int D, int CK>
__global__ __launch_bounds__(DELTA_LPR * DELTA_ROWS) void k_deltanet(const DeltaArgs a) {
  constexpr int RW = DELTA_ROWS, R = D / RW, LPR = DELTA_LPR, NT = LPR * RW, NW = NT / 64, PER = D / LPR;
  constexpr int ROW = D + 4 * LPR;  // LDS row of q or k: the row parts padded apart by 4 floats (distinct banks)
  constexpr int M = CK - 1;    // window length
  static_assert(D % RW == 0, "head size is a multiple of the rows per workgroup");
  constexpr int NCH = 2 * D + RW;      // channels of the workgroup: the head's q and k, then its RW rows of v
  constexpr int EXT = M + DELTA_MAX_B;  // per channel: the window (oldest first), then the launch's inputs
  __shared__ float cq[DELTA_MAX_B * ROW], ck[DELTA_MAX_B * ROW], cv[DELTA_MAX_B * RW];
  __shared__ float ext[NCH * EXT], wts[NCH * CK];
  __shared__ double gexp[DELTA_MAX_B], bet[DELTA_MAX_B];
  const int hv = blockIdx.x / R, r = blockIdx.x - hv * R, kh = hv % a.nK, tid = threadIdx.x, lane = tid & 63,
            wave = tid >> 6;
  const int B = a.B;
  auto pidx = [](int i) { return i + (i / PER) * 4; };
  const int keyDim = a.nK * D;
  // channel c of the workgroup: group (0 q, 1 k, 2 v), index within the head, conv channel, window
  auto chan = [&](int c, int &grp, int &i) {
    grp = c < D ? 0 : c < 2 * D ? 1 : 2;
    i = grp < 2 ? c - grp * D : r * RW + (c - 2 * D);
    return grp == 0 ? kh * D + i : grp == 1 ? keyDim + kh * D + i : 2 * keyDim + hv * D + i;
  };

  // lane (j, p) holds S[jg][p*PER .. p*PER+PER) of the head's row jg = r RW + j (requested first: it is used last)
  const int j = tid / LPR, p = tid % LPR, jg = r * RW + j;
  float S[PER];
  float *srow = a.ssm + ((long)hv * D + jg) * D + p * PER;
  #pragma unroll
  for (int c = 0; c < PER; c += 4) {
    const float4 v4 = *(const float4 *)(srow + c);
    S[c] = v4.x; S[c + 1] = v4.y; S[c + 2] = v4.z; S[c + 3] = v4.w;
  }

  // ---- stage the windows, the B inputs and the conv weights of the workgroup's channels (every load issued up front)
  {
    // all loads first (registers), then the LDS stores: a load per loop iteration would wait out its latency each time
    constexpr int SE = ((M + DELTA_MAX_B) * NCH + NT - 1) / NT, SW = (CK * NCH + NT - 1) / NT;
    float ve[SE], vw[SW];
    #pragma unroll
    for (int k = 0; k < SE; k++) {
      const int idx = tid + k * NT, t = idx / NCH, c = idx - t * NCH;
      int grp, i;
      const int ch = chan(c, grp, i);
      ve[k] = idx >= (M + B) * NCH ? 0.f
              : t < M ? a.conv[(((long)hv * 3 + grp) * D + i) * M + t] : a.qkv[(long)(t - M) * a.ldqkv + ch];
    }
    #pragma unroll
    for (int k = 0; k < SW; k++) {
      const int idx = tid + k * NT, t = idx / NCH, c = idx - t * NCH;
      int grp, i;
      const int ch = chan(c, grp, i);
      vw[k] = idx < CK * NCH ? a.convW[(long)ch * CK + t] : 0.f;
    }
    #pragma unroll
    for (int k = 0; k < SE; k++) {
      const int idx = tid + k * NT, t = idx / NCH, c = idx - t * NCH;
      if (idx < (M + B) * NCH) ext[c * EXT + t] = ve[k];
    }
    #pragma unroll
    for (int k = 0; k < SW; k++) {
      const int idx = tid + k * NT, t = idx / NCH, c = idx - t * NCH;
      if (idx < CK * NCH) wts[c * CK + t] = vw[k];
    }
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

  // ---- conv + SiLU (convStep, src/compute/ref-deltanet.js:42-55) of every (channel, token): the window of token b is
  // ext[b .. b + M), its input ext[b + M]; f64 products added in window order, then the input's
  #pragma unroll 2
  for (int idx = tid; idx < B * NCH; idx += NT) {
    const int b = idx / NCH, c = idx - b * NCH;
    int grp, i;
    chan(c, grp, i);
    const float *e = ext + c * EXT + b, *w = wts + c * CK;
    double acc = 0.0;
    #pragma unroll
    for (int t = 0; t < M; t++) acc += (double)w[t] * (double)e[t];
    acc += (double)w[M] * (double)e[M];
    if (a.capConv && (grp == 2 || r == 0)) {  // the window after token b (q and k by the head's first workgroup)
      float *cw = a.capConv + (long)b * a.capStride + (((long)hv * 3 + grp) * D + i) * M;
      #pragma unroll
      for (int t = 0; t < M; t++) cw[t] = e[t + 1];
    }
    const float y = (float)(acc / (1.0 + exp(-acc)));
    if (grp == 0) cq[b * ROW + pidx(i)] = y;
    else if (grp == 1) ck[b * ROW + pidx(i)] = y;
    else cv[b * RW + (i - r * RW)] = y;
  }
  for (int idx = tid; idx < RW * M; idx += NT) {  // the v windows of the workgroup's rows after the last token
    const int c = 2 * D + idx / M, t = idx - (idx / M) * M;
    int grp, i;
    chan(c, grp, i);
    a.conv[(((long)hv * 3 + grp) * D + i) * M + t] = ext[c * EXT + B + t];
  }
  __syncthreads();

  // ---- L2 norms (l2normHeads, src/compute/ref-deltanet.js:61-69): one wave per (token, q or k) row
  // (two rows per wave at a time, rr and rr + NW, as independent chains)
  for (int rr = wave; rr < 2 * B; rr += 2 * NW) {
    const int r1 = rr + NW < 2 * B ? rr + NW : rr;
    float *row0 = ((rr & 1) ? ck : cq) + (rr >> 1) * ROW, *row1 = ((r1 & 1) ? ck : cq) + (r1 >> 1) * ROW;
    double s0 = 0.0, s1 = 0.0;
    for (int i = lane; i < D; i += 64) {
      const double x0 = (double)row0[pidx(i)], x1 = (double)row1[pidx(i)];
      s0 += x0 * x0;
      s1 += x1 * x1;
    }
    s0 = wave_sum_xor(s0, 64);
    s1 = wave_sum_xor(s1, 64);
    const double f0 = ((rr & 1) ? 1.0 : 1.0 / sqrt((double)D)) / sqrt(s0 + a.eps);
    const double f1 = ((r1 & 1) ? 1.0 : 1.0 / sqrt((double)D)) / sqrt(s1 + a.eps);
    for (int i = lane; i < D; i += 64) {
      const float y0 = (float)((double)row0[pidx(i)] * f0), y1 = (float)((double)row1[pidx(i)] * f1);
      row0[pidx(i)] = y0;
      if (r1 != rr) row1[pidx(i)] = y1;
    }
  }
  __syncthreads();

  // ---- delta rule (deltaRuleHead, src/compute/ref-deltanet.js:86-96) on the lane's part of row jg
  for (int b = 0; b < B; b++) {
    const double g = gexp[b], be = bet[b];
    const float *kp = ck + b * ROW + p * (PER + 4), *qp = cq + b * ROW + p * (PER + 4);
    double sk = 0.0;
    #pragma unroll
    for (int c = 0; c < PER; c++) { const double s = (double)S[c] * g; S[c] = (float)s; sk += s * (double)kp[c]; }
    sk += __shfl_xor(sk, 1);  // ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)) on all eight lanes of the row
    sk += __shfl_xor(sk, 2);
    sk += __shfl_xor(sk, 4);
    const double d = ((double)cv[b * RW + j] - sk) * be;
    double o = 0.0;
    #pragma unroll
    for (int c = 0; c < PER; c++) { const double s = (double)S[c] + (double)kp[c] * d; S[c] = (float)s; o += s * (double)qp[c]; }
    o += __shfl_xor(o, 1);
    o += __shfl_xor(o, 2);
    o += __shfl_xor(o, 4);
    if (p == 0) a.xcore[((long)hv * DELTA_MAX_B + b) * D + jg] = (float)o;  // (for k_delta_norm)
    if (a.capSsm) {  // the state after token b
      float *cs = a.capSsm + (long)b * a.capStride + ((long)hv * D + jg) * D + p * PER;
      #pragma unroll
      for (int c = 0; c < PER; c++) __builtin_nontemporal_store(S[c], cs + c);
    }
  }
  // the state and its captures with nontemporal stores: they are read only by later launches
  #pragma unroll
  for (int c = 0; c < PER; c++) __builtin_nontemporal_store(S[c], srow + c);
}

// The gated RMSNorm (gatedRmsNormHead, src/compute/ref-deltanet.js:102-106) + quantisation of one value head's B output
// rows, one wave per token (the wave's tokens in pairs k, k + 1, their scales as independent chains), and the head's q
// and k conv windows after the last token: the last M of [the window k_deltanet read, the launch's B inputs].
template <int D, int CK>
__global__ __launch_bounds__(256) void k_delta_norm(const DeltaArgs a) {
  constexpr int NW = 4, M = CK - 1, ZB = ((DELTA_MAX_B + NW - 1) / NW + 1) / 2 * 2, ZI = (D + 63) / 64;
  __shared__ float core[DELTA_MAX_B * D];
  const int hv = blockIdx.x, kh = hv % a.nK, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, B = a.B;
  const int keyDim = a.nK * D;
  // every load first: the rows, the gate values and norm weights of the lane's outputs (token wave + NW k, value
  // 64 q + lane), the window sources of the thread's q / k channel
  constexpr int XJ = (DELTA_MAX_B * D + 255) / 256;
  float xv[XJ];
  #pragma unroll
  for (int k = 0; k < XJ; k++) {
    const int idx = tid + 256 * k;
    xv[k] = a.xcore[(long)hv * DELTA_MAX_B * D + (idx < B * D ? idx : 0)];
  }
  float zr[ZB][ZI], nwr[ZI];
  #pragma unroll
  for (int q = 0; q < ZI; q++) {
    const int i = 64 * q + lane;
    nwr[q] = a.normW[i < D ? i : 0];
    #pragma unroll
    for (int k = 0; k < ZB; k++) {
      const int b = wave + NW * k;
      zr[k][q] = a.z[(long)(b < B ? b : 0) * a.ldz + hv * D + (i < D ? i : 0)];
    }
  }
  constexpr int WJ = (2 * D + 255) / 256;
  float wv[WJ][M];
  #pragma unroll
  for (int k = 0; k < WJ; k++) {
    const int c = tid + 256 * k, grp = c < D ? 0 : 1, i = c < 2 * D ? c - grp * D : 0;
    const int ch = grp == 0 ? kh * D + i : keyDim + kh * D + i;
    #pragma unroll
    for (int t = 0; t < M; t++) {
      const int u = B + t;  // position in [window (M), inputs (B)]
      wv[k][t] = u < M ? a.conv[(((long)hv * 3 + grp) * D + i) * M + u] : a.qkv[(long)(u - M) * a.ldqkv + ch];
    }
  }
  #pragma unroll
  for (int k = 0; k < XJ; k++) {
    const int idx = tid + 256 * k;
    if (idx < B * D) core[idx] = xv[k];
  }
  #pragma unroll
  for (int k = 0; k < WJ; k++) {
    const int c = tid + 256 * k, grp = c < D ? 0 : 1, i = c - grp * D;
    if (c < 2 * D) {
      #pragma unroll
      for (int t = 0; t < M; t++) a.conv[(((long)hv * 3 + grp) * D + i) * M + t] = wv[k][t];
    }
  }
  __syncthreads();
  #pragma unroll
  for (int k = 0; k < ZB; k += 2) {
    const int b0 = wave + NW * k;
    if (b0 >= B) break;
    const int b1 = b0 + NW < B ? b0 + NW : b0;
    const float *o0 = core + b0 * D, *o1 = core + b1 * D;
    double s0 = 0.0, s1 = 0.0;
    for (int i = lane; i < D; i += 64) {
      const double x0 = (double)o0[i], x1 = (double)o1[i];
      s0 += x0 * x0;
      s1 += x1 * x1;
    }
    s0 = wave_sum_xor(s0, 64);
    s1 = wave_sum_xor(s1, 64);
    const double f[2] = {1.0 / sqrt(s0 / (double)D + a.eps), 1.0 / sqrt(s1 / (double)D + a.eps)};
    #pragma unroll
    for (int h = 0; h < 2; h++) {
      const int b = h ? b1 : b0;
      if (h && b1 == b0) break;
      #pragma unroll
      for (int q = 0; q < ZI; q++) {
        const int i = 64 * q + lane;
        if (i < D) {  // D = 32: lanes 32-63 idle, a whole 32-lane block group
          const double zz = (double)zr[k + h][q];
          const float v = (float)((double)core[b * D + i] * f[h] * (double)nwr[q] * (zz / (1.0 + exp(-zz))));
          const int col = hv * D + i;
          if (a.out) a.out[(long)b * a.ldo + col] = v;
          quant_block32(v, col, a.act, b);
        }
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
  ZL_REQUIRE(a0.xcore, ZL_ERR_ARG, "Gated DeltaNet: output row buffer missing");
  for (int t0 = 0; t0 < a0.B; t0 += DELTA_MAX_B) {
    DeltaArgs a = a0;
    a.B = std::min(DELTA_MAX_B, a0.B - t0);
    a.qkv += (long)t0 * a.ldqkv;
    a.z += (long)t0 * a.ldz;
    a.alpha += (long)t0 * a.ldab;
    a.beta += (long)t0 * a.ldab;
    a.act = act_rows(a0.act, t0);
    if (a.out) a.out += (long)t0 * a.ldo;
    const dim3 grid((unsigned)(a.nV * (D / DELTA_ROWS))), blk(DELTA_LPR * DELTA_ROWS), gn((unsigned)a.nV), bn(256);
    if (D == 128) {
      hipLaunchKernelGGL((k_deltanet<128, 4>), grid, blk, 0, st, a);
      hipLaunchKernelGGL((k_delta_norm<128, 4>), gn, bn, 0, st, a);
    } else if (D == 64) {
      hipLaunchKernelGGL((k_deltanet<64, 4>), grid, blk, 0, st, a);
      hipLaunchKernelGGL((k_delta_norm<64, 4>), gn, bn, 0, st, a);
    } else {
      hipLaunchKernelGGL((k_deltanet<32, 4>), grid, blk, 0, st, a);
      hipLaunchKernelGGL((k_delta_norm<32, 4>), gn, bn, 0, st, a);
    }
    ZL_HIP(hipGetLastError());
  }
}

}  // namespace zl
