// Multi-token prefill for the GPT-2 program on gfx950: the P prompt positions
// of all B rows go through each layer together (M = B * P rows), so the
// projections are matrix products on the matrix cores instead of P decode
// steps. Appended to the prelude (hip/prelude.h, VBLOCK 256) and compiled at
// run time by hipRTC.
//
// Row m of every activation buffer is position p = m % P of batch row
// b = m / P, at sequence position t0 + p, t0 read from the device (the
// model's position counter, advanced by P at the end). Activations are fp32
// [M, width]; the key/value cache is the decode kernel's [B, L, tmax, H, 64]
// fp16. Positions at or past tmax write no cache row and attend to rows
// 0 .. tmax - 1 only.
//
// Arithmetic follows the program's statements (fp16 weights, fp32 math, the
// cache rounded to fp16 before attention reads it); products run on
// v_mfma_f32_16x16x32_f16 with every activation split into two fp16 halves
// (hi + lo / 2048: 22 significant bits at any magnitude), each half's products
// accumulated in fp32 on its own and combined at the end.

#define PF_E 64                 // head width
#define PF_TILE 32              // output tile of one block: 32 rows x 32 columns

// ---------------------------------------------------------------- embedding
// Z[m] = wte[tok[m]] + wpe[t0 + p]   (gpt2.vst Q1; ids and positions
// clamped into their tables). One block per row.
extern "C" __global__ __launch_bounds__(256) void pf_embed(const int* __restrict__ tok, int P,
                                                            const int* __restrict__ tp,
                                                            const vh_half* __restrict__ wte,
                                                            const vh_half* __restrict__ wpe, float* __restrict__ Z,
                                                            int D, int V, int npos) {
  const int m = blockIdx.x;
  int x = tok[m];
  x = x < 0 ? 0 : (x >= V ? V - 1 : x);
  int pos = *tp + m % P;
  pos = pos < 0 ? 0 : (pos >= npos ? npos - 1 : pos);
  for (int i = threadIdx.x; i < D; i += blockDim.x)
    Z[(size_t)m * D + i] = h2f(wte[(size_t)x * D + i]) + h2f(wpe[(size_t)pos * D + i]);
}

// ---------------------------------------------------------------- layer norm
// Y[i] = (X[r] - mean) / sqrt(var + 1e-5) * w + b for r = row0 + i * rstride
// (biased variance; mean and variance as sums of x / D and (x - mean)^2 / D,
// as gpt2.vst Q2 writes them). One block per output row; D <= 8 * 256.
extern "C" __global__ __launch_bounds__(256) void pf_ln(const float* __restrict__ X, int row0, int rstride,
                                                         const vh_half* __restrict__ w, const vh_half* __restrict__ b,
                                                         float* __restrict__ Y, int D) {
  __shared__ float red[VNWAVE];
  const float* x = X + (size_t)(row0 + (size_t)blockIdx.x * rstride) * D;
  float* y = Y + (size_t)blockIdx.x * D;
  const float fd = (float)D;
  float v[8];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = threadIdx.x + j * 256;
    v[j] = i < D ? x[i] : 0.0f;
    if (i < D) s += v[j] / fd;
  }
  const float mean = block_red_sum(s, red);
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = threadIdx.x + j * 256;
    if (i < D) q += (v[j] - mean) * (v[j] - mean) / fd;
  }
  vh_lds_sync();
  const float var = block_red_sum(q, red);
  const float sd = sqrtf(var + 0.00001f);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = threadIdx.x + j * 256;
    if (i < D) y[i] = (v[j] - mean) / sd * h2f(w[i]) + h2f(b[i]);
  }
}

// ---------------------------------------------------------------- products
// C = A Wt^T over K (A fp32 [M, K] with row stride lda, Wt fp16 [N, K], the
// transposed weight: row n holds output n's weights contiguously), then the
// epilogue of `mode`:
//   0  out[m, n] = C + bias[n]                       (plain; bias optional)
//   1  out[m, n] = (out[m, n] + C) + bias[n]          (residual add, in place)
//   2  out[m, n] = gelu_tanh(C + bias[n])             (feed-forward widening)
//   3  qkv: n < D -> out[m, n] (queries); D <= n < 2D -> key cache;
//      2D <= n -> value cache, at this row's sequence position (fp16)
// A block computes a 32 x 32 tile as 2 x 2 matrix-core tiles; its four waves
// take every fourth 32-deep step of K (a multiple of 32) and their partial
// tiles are added through LDS in wave order, so results do not depend on
// timing. Consecutive blocks take consecutive column tiles of one row band.
__device__ __forceinline__ float pf_gelu(float u) {
  return 0.5f * u * (1.0f + tanhf(0.7978845608028654f * (u + 0.044715f * u * u * u)));
}

#ifndef PF_UNROLL
#define PF_UNROLL 2              // k-steps whose loads are issued together (2: measured best of 2, 4, 8)
#endif

__device__ __forceinline__ void pf_load_a(const float* __restrict__ A, int lda, int row, int M, int k,
                                          vh_f32x4& x0, vh_f32x4& x1) {
  if (row < M) {
    x0 = *(const vh_f32x4*)(A + (size_t)row * lda + k);
    x1 = *(const vh_f32x4*)(A + (size_t)row * lda + k + 4);
  } else {
    x0 = x1 = vh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
}

__device__ __forceinline__ void pf_split_a(vh_f32x4 x0, vh_f32x4 x1, vh_u32x4& hi, vh_u32x4& lo) {
  const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  vh_split8s(v, hi, lo);
}

// The epilogue of one output value c = C[m, n] (modes above).
__device__ __forceinline__ void pf_epi(int mode, int m, int n, float c, const vh_half* __restrict__ bias, int N,
                                       float* __restrict__ out, int ldo, vh_half* __restrict__ kc,
                                       vh_half* __restrict__ vc, int P, const int* __restrict__ tp, int layer,
                                       int L, int tmax) {
  const float bn = bias ? h2f(bias[n]) : 0.0f;
  if (mode == 0) {
    out[(size_t)m * ldo + n] = c + bn;
  } else if (mode == 1) {
    float* o = out + (size_t)m * ldo + n;
    *o = (*o + c) + bn;
  } else if (mode == 2) {
    out[(size_t)m * ldo + n] = pf_gelu(c + bn);
  } else {
    const int D = N / 3;
    const float val = c + bn;
    if (n < D) {
      out[(size_t)m * ldo + n] = val;
    } else {
      const int b = m / P, pos = *tp + m % P;
      if (pos >= 0 && pos < tmax) {
        const size_t at = ((size_t)(b * L + layer) * tmax + pos) * D + (n % D);
        (n < 2 * D ? kc : vc)[at] = f2h(val);
      }
    }
  }
}

// `ksplit` > 1 splits K over blocks as well: block b makes part b / tiles of
// the fold for tile b % tiles and stores its partial tile in ws[part][m][n];
// pf_reduce then adds the parts in part order and applies the epilogue.
extern "C" __global__ __launch_bounds__(256) void pf_gemm(
    const float* __restrict__ A, int lda, const vh_half* __restrict__ Wt, const vh_half* __restrict__ bias,
    int M, int N, int K, int mode, float* __restrict__ out, int ldo,
    vh_half* __restrict__ kc, vh_half* __restrict__ vc, int P, const int* __restrict__ tp, int layer, int L,
    int tmax, int ksplit, float* __restrict__ ws) {
  __shared__ vh_f32x4 part[VNWAVE][2][2][2][64];     // [wave][hi/lo][i][j][lane]
  const int ntn = (N + PF_TILE - 1) / PF_TILE, ntm = (M + PF_TILE - 1) / PF_TILE;
  const int tile = blockIdx.x % (ntn * ntm), kp = blockIdx.x / (ntn * ntm);
  const int tn = tile % ntn, tm = tile / ntn;
  const int nks = K / 32, ks0 = kp * nks / ksplit, ks1 = (kp + 1) * nks / ksplit;
  const int kend = 32 * ks1;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m0 = tm * PF_TILE, n0 = tn * PF_TILE;
  const int r = lane & 15, kq = (lane >> 4) * 8;
  vh_f32x4 acc[2][2], acl[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = acl[i][j] = vh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int c0 = n0 + r, c1 = n0 + 16 + r;
  const vh_half* w0 = Wt + (size_t)(c0 < N ? c0 : 0) * K;
  const vh_half* w1 = Wt + (size_t)(c1 < N ? c1 : 0) * K;
  for (int k0 = 32 * (ks0 + wave); k0 < kend; k0 += 32 * VNWAVE * PF_UNROLL) {
    vh_f32x4 xa[PF_UNROLL][2][2];
    vh_u32x4 bw[PF_UNROLL][2];
#pragma unroll
    for (int u = 0; u < PF_UNROLL; ++u) {
      const int ks = k0 + 32 * VNWAVE * u;
      const int k = ks + kq;
      const bool in = ks < kend;
      pf_load_a(A, lda, in ? m0 + r : M, M, k, xa[u][0][0], xa[u][0][1]);
      pf_load_a(A, lda, in ? m0 + 16 + r : M, M, k, xa[u][1][0], xa[u][1][1]);
      bw[u][0] = in && c0 < N ? ld16(w0 + k) : vh_u32x4{0u, 0u, 0u, 0u};
      bw[u][1] = in && c1 < N ? ld16(w1 + k) : vh_u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < PF_UNROLL; ++u) {
      if (k0 + 32 * VNWAVE * u >= kend) break;
      vh_u32x4 ah[2], al[2];
      pf_split_a(xa[u][0][0], xa[u][0][1], ah[0], al[0]);
      pf_split_a(xa[u][1][0], xa[u][1][1], ah[1], al[1]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = vh_mfma(ah[i], bw[u][j], acc[i][j]);
          acl[i][j] = vh_mfma(al[i], bw[u][j], acl[i][j]);
        }
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      part[wave][0][i][j][lane] = acc[i][j];
      part[wave][1][i][j][lane] = acl[i][j];
    }
  vh_lds_sync();
  // wave w finishes matrix-core tile (i, j) = (w / 2, w % 2)
  const int i = wave >> 1, j = wave & 1;
  vh_f32x4 hi = part[0][0][i][j][lane], lo = part[0][1][i][j][lane];
#pragma unroll
  for (int w = 1; w < VNWAVE; ++w) {
    hi += part[w][0][i][j][lane];
    lo += part[w][1][i][j][lane];
  }
  const int n = n0 + 16 * j + r;
  if (n >= N) return;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int m = m0 + 16 * i + 4 * (lane >> 4) + v;
    if (m >= M) continue;
    const float c = fmaf(lo[v], 1.0f / VH_LO_SCALE, hi[v]);
    if (ksplit > 1)
      ws[((size_t)kp * M + m) * N + n] = c;
    else
      pf_epi(mode, m, n, c, bias, N, out, ldo, kc, vc, P, tp, layer, L, tmax);
  }
}

// The parts of a split product added in part order, then the epilogue. One
// thread per output value.
extern "C" __global__ __launch_bounds__(256) void pf_reduce(
    const float* __restrict__ ws, int ksplit, const vh_half* __restrict__ bias, int M, int N, int mode,
    float* __restrict__ out, int ldo, vh_half* __restrict__ kc, vh_half* __restrict__ vc, int P,
    const int* __restrict__ tp, int layer, int L, int tmax) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (size_t)M * N) return;
  const int m = (int)(e / N), n = (int)(e % N);
  float c = ws[e];
  for (int k = 1; k < ksplit; ++k) c += ws[(size_t)k * M * N + e];
  pf_epi(mode, m, n, c, bias, N, out, ldo, kc, vc, P, tp, layer, L, tmax);
}

// ---------------------------------------------------------------- attention
// One wave per (row m, head h): scores of the query against cache positions
// 0 .. t0 + p (gpt2.vst Q5: dot over e, divided by 8), the max-subtracted
// softmax (Q6), and the weighted values (Q7), read from the fp16 cache the
// qkv product just wrote. O[m, h * 64 + e] receives the head's output.
// `ws` holds each wave's scores, then weights, for up to PF_TMAX positions.
extern "C" __global__ __launch_bounds__(256) void pf_attn(const float* __restrict__ Q, const vh_half* __restrict__ kc,
                                                           const vh_half* __restrict__ vc, float* __restrict__ O,
                                                           int M, int P, const int* __restrict__ tp, int layer,
                                                           int L, int tmax, int H) {
  __shared__ float qs[VNWAVE][PF_E];
  __shared__ float ws[VNWAVE][PF_TMAX];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int item = blockIdx.x * VNWAVE + wave;
  const bool live = item < M * H;
  const int m = live ? item / H : 0, h = live ? item % H : 0;
  const int D = H * PF_E;
  const int b = m / P, at = *tp + m % P;
  const int pos = at < tmax ? at : tmax - 1;
  const size_t base = (size_t)(b * L + layer) * tmax * D + (size_t)h * PF_E;
  if (live) qs[wave][lane] = Q[(size_t)m * D + h * PF_E + lane];
  vh_lds_sync();
  float mx = -INFINITY;
  if (live) {
    for (int s = lane; s <= pos; s += 64) {
      const vh_half* kr = kc + base + (size_t)s * D;
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < PF_E; e += 8) {
        float kv[8];
        unpack8(ld16(kr + e), kv);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = fmaf(qs[wave][e + j], kv[j], acc);
      }
      const float sc = acc * 0.125f;      // / 8, exact
      ws[wave][s] = sc;
      mx = fmaxf(mx, sc);
    }
  }
  mx = wave_red_max(mx);
  float sum = 0.0f;
  if (live) {
    for (int s = lane; s <= pos; s += 64) {
      const float ex = expf(ws[wave][s] - mx);
      ws[wave][s] = ex;
      sum += ex;
    }
  }
  sum = wave_red_sum(sum);
  if (live) {
    for (int s = lane; s <= pos; s += 64) ws[wave][s] = ws[wave][s] / sum;
  }
  vh_lds_sync();
  if (live) {
    float o = 0.0f;
    for (int s = 0; s <= pos; ++s) o = fmaf(ws[wave][s], h2f(vc[base + (size_t)s * D + lane]), o);
    O[(size_t)m * D + h * PF_E + lane] = o;
  }
}

// ---------------------------------------------------------------- argmax
// Per row of logits [B, V]: the largest value, a tie to the lowest id
// (gpt2.vst Q10). Writes the token into x (the next step's input) and, as a
// float, into `next`; block 0 advances the position counter by P. One block
// per row.
extern "C" __global__ __launch_bounds__(256) void pf_argmax(const float* __restrict__ logit, int V,
                                                             int* __restrict__ x, float* __restrict__ next,
                                                             int* __restrict__ tp, int P) {
  __shared__ float rv[VNWAVE];
  __shared__ int ri[VNWAVE];
  const float* lg = logit + (size_t)blockIdx.x * V;
  float best = -INFINITY;
  int id = V;
  for (int n = threadIdx.x; n < V; n += blockDim.x) argmax_pair(best, id, lg[n], n);
  block_argmax(best, id, rv, ri);
  if (threadIdx.x == 0) {
    x[blockIdx.x] = id;
    next[blockIdx.x] = (float)id;
    if (blockIdx.x == 0) *tp += P;     // the last kernel of a pass: advance the position
  }
}
