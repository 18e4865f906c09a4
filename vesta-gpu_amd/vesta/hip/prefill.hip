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
#define PF_TILE 64              // output tile of one block: 64 rows x 64 columns
#define PF_BK 64                // fold chunk staged in LDS per step of a block
#define PF_LDA (PF_BK + 8)      // LDS row pitch of staged operands in halves (16 bytes of padding)

// ---------------------------------------------------------------- embedding
// Z[m] = wte[tok[m]] + wpe[t0 + p]   (gpt2.vst Q1; ids and positions
// clamped into their tables). One block per row, thread t on the eight
// consecutive values 8t .. 8t + 7 (D <= 8 * 256).
extern "C" __global__ __launch_bounds__(256) void pf_embed(const int* __restrict__ tok, int P,
                                                            const int* __restrict__ tp,
                                                            const vh_half* __restrict__ wte,
                                                            const vh_half* __restrict__ wpe, float* __restrict__ Z,
                                                            int D, int V, int npos) {
  const int m = blockIdx.x, k8 = 8 * threadIdx.x;
  int x = tok[m];
  x = x < 0 ? 0 : (x >= V ? V - 1 : x);
  int pos = *tp + m % P;
  pos = pos < 0 ? 0 : (pos >= npos ? npos - 1 : pos);
  if (k8 >= D) return;
  float a[8], b[8];
  unpack8(ld16(wte + (size_t)x * D + k8), a);
  unpack8(ld16(wpe + (size_t)pos * D + k8), b);
  float* z = Z + (size_t)m * D + k8;
  *(vh_f32x4*)z = vh_f32x4{a[0] + b[0], a[1] + b[1], a[2] + b[2], a[3] + b[3]};
  *(vh_f32x4*)(z + 4) = vh_f32x4{a[4] + b[4], a[5] + b[5], a[6] + b[6], a[7] + b[7]};
}

// ---------------------------------------------------------------- fragment order
// The decode products (pf_mgemm*, at most 64 rows) read both operands in the
// order the matrix cores take them (v_mfma_f32_16x16x32_f16: lane l = 16 q + r
// holds row r, fold positions 8 q .. 8 q + 7 of a 16 x 32 operand tile), so
// that each operand load of a wave is one contiguous kilobyte:
//   weights      Wf[n-tile][k-step][lane][8]         n = 16 n-tile + r
//   activations  Af[plane][m-tile][k-step][lane][8]  m = 16 m-tile + r
// with k = 32 k-step + 8 q + e; plane 0 holds the nearest fp16 (hi), plane 1
// the remainder scaled by 2^11 (vh_split8s). MT m-tiles, KT k-steps; rows
// past the last real one are never written and only reach discarded outputs.
// A producer of an activation row stores eight values k8 .. k8 + 7 (k8 a
// multiple of 8) of row m at once; `bad` is raised for a value beyond the
// fp16 range.
__device__ __forceinline__ void pf_frag_put8(vh_half* __restrict__ F, int MT, int KT, int m, int k8, const float* v,
                                             bool& bad) {
  bad |= vh_beyond_half8(v);
  vh_u32x4 hi, lo;
  vh_split8s(v, hi, lo);
  const size_t at = (((size_t)(m >> 4) * KT + (k8 >> 5)) * 64 + ((k8 >> 3) & 3) * 16 + (m & 15)) * 8;
  *(vh_u32x4*)(F + at) = hi;
  *(vh_u32x4*)(F + (size_t)MT * KT * 512 + at) = lo;
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
// A block computes a 64 x 64 tile. The fold goes in chunks of 64 staged in
// LDS (double-buffered: the next chunk's global loads are in flight while
// one chunk is multiplied): A as fp16 halves (hi, and the remainder scaled by
// 2^11), Wt as loaded. Wave w multiplies row tile w by the four column tiles,
// hi and lo halves into separate accumulators. K is a multiple of 64.
// gelu_tanh(u) = 0.5 u (1 + tanh(y)), y = 0.7978845608028654 (u + 0.044715 u^3),
// evaluated as u / (1 + exp(-2 y)) (0.5 (1 + tanh y) is the logistic function
// of 2 y): one exponential and one division instead of tanh; in fp32 its
// error against the exact function is that of the tanh form (5e-7 absolute
// over |u| <= 12 for either).
__device__ __forceinline__ float pf_gelu(float u) {
  const float y = 0.7978845608028654f * (u + 0.044715f * u * u * u);
  return u / (1.0f + __expf(-2.0f * y));
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

// One chunk's global loads: thread t takes float4 f = t + 256 i of A
// (row f / 16, columns 4 (f % 16)..+4) and 16-byte piece g = t + 256 i of Wt
// (row g / 8, columns 8 (g % 8)..+8); rows past M or N read as zero.
struct PfChunk {
  vh_f32x4 a[4];
  vh_u32x4 w[2];
};

__device__ __forceinline__ void pf_chunk_load(PfChunk& c, const float* __restrict__ A, int lda,
                                              const vh_half* __restrict__ Wt, int M, int N, int K, int m0, int n0,
                                              int k0) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = t + 256 * i, row = m0 + (f >> 4), col = k0 + 4 * (f & 15);
    c.a[i] = row < M ? *(const vh_f32x4*)(A + (size_t)row * lda + col) : vh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int g = t + 256 * i, n = n0 + (g >> 3), col = k0 + 8 * (g & 7);
    c.w[i] = n < N ? ld16(Wt + (size_t)n * K + col) : vh_u32x4{0u, 0u, 0u, 0u};
  }
}

// The chunk into LDS: A rows as hi / lo fp16 halves, Wt rows as they are.
// `bad` is raised when an A value is beyond the fp16 range (see vh_beyond_half8).
__device__ __forceinline__ void pf_chunk_store(const PfChunk& c, vh_half* ah, vh_half* al, vh_half* wl, bool& bad) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = t + 256 * i, row = f >> 4, col = 4 * (f & 15);
    const float v[4] = {c.a[i].x, c.a[i].y, c.a[i].z, c.a[i].w};
    _Float16 h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bad |= !(__builtin_fabsf(v[j]) <= VH_HALF_MAX);
      h[j] = (_Float16)v[j];
      l[j] = (_Float16)((v[j] - (float)h[j]) * VH_LO_SCALE);
    }
    *(vh_u32x2*)(ah + row * PF_LDA + col) = vh_u32x2{
        (unsigned)__builtin_bit_cast(unsigned short, h[0]) | ((unsigned)__builtin_bit_cast(unsigned short, h[1]) << 16),
        (unsigned)__builtin_bit_cast(unsigned short, h[2]) | ((unsigned)__builtin_bit_cast(unsigned short, h[3]) << 16)};
    *(vh_u32x2*)(al + row * PF_LDA + col) = vh_u32x2{
        (unsigned)__builtin_bit_cast(unsigned short, l[0]) | ((unsigned)__builtin_bit_cast(unsigned short, l[1]) << 16),
        (unsigned)__builtin_bit_cast(unsigned short, l[2]) | ((unsigned)__builtin_bit_cast(unsigned short, l[3]) << 16)};
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int g = t + 256 * i, n = g >> 3, col = 8 * (g & 7);
    *(vh_u32x4*)(wl + n * PF_LDA + col) = c.w[i];
  }
}

// One staged chunk (PF_BK deep) multiplied into wave `wave`'s row tile: the
// hi and lo halves of A against the four column tiles of Wt.
__device__ __forceinline__ void pf_chunk_mma(vh_half (*buf)[PF_TILE * PF_LDA], int wave, int r, int kq,
                                             vh_f32x4* acc, vh_f32x4* acl) {
#pragma unroll
  for (int ks = 0; ks < PF_BK; ks += 32) {
    const int k = ks + kq;
    const vh_u32x4 ah = *(const vh_u32x4*)(buf[0] + (16 * wave + r) * PF_LDA + k);
    const vh_u32x4 al = *(const vh_u32x4*)(buf[1] + (16 * wave + r) * PF_LDA + k);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const vh_u32x4 b = *(const vh_u32x4*)(buf[2] + (16 * j + r) * PF_LDA + k);
      acc[j] = vh_mfma(ah, b, acc[j]);
      acl[j] = vh_mfma(al, b, acl[j]);
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
    int tmax, int ksplit, float* __restrict__ ws, unsigned* __restrict__ err) {
  __shared__ __attribute__((aligned(16))) vh_half lds[2][3][PF_TILE * PF_LDA];   // [buffer][hi, lo, Wt]
  const int ntn = (N + PF_TILE - 1) / PF_TILE, ntm = (M + PF_TILE - 1) / PF_TILE;
  const int tile = blockIdx.x % (ntn * ntm), kp = blockIdx.x / (ntn * ntm);
  const int tn = tile % ntn, tm = tile / ntn;
  const int m0 = tm * PF_TILE, n0 = tn * PF_TILE;
  const int nch = K / PF_BK, c0 = kp * nch / ksplit, c1 = (kp + 1) * nch / ksplit;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, kq = (lane >> 4) * 8;
  vh_f32x4 acc[4], acl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = acl[j] = vh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // Chunks go global -> registers -> LDS three deep: while chunk c is
  // multiplied out of one LDS buffer, chunk c + 1 waits in registers for the
  // other buffer and chunk c + 2 is in flight into a second register stage.
  // (Unrolled by two so each register stage keeps its own name.)
  PfChunk r0, r1;
  bool bad = false;
  if (c0 < c1) {
    pf_chunk_load(r0, A, lda, Wt, M, N, K, m0, n0, c0 * PF_BK);
    pf_chunk_store(r0, lds[0][0], lds[0][1], lds[0][2], bad);
  }
  if (c0 + 1 < c1) pf_chunk_load(r0, A, lda, Wt, M, N, K, m0, n0, (c0 + 1) * PF_BK);
  if (c0 + 2 < c1) pf_chunk_load(r1, A, lda, Wt, M, N, K, m0, n0, (c0 + 2) * PF_BK);
  vh_lds_sync();
  for (int c = c0; c < c1; c += 2) {
    pf_chunk_mma(lds[0], wave, r, kq, acc, acl);
    if (c + 1 < c1) pf_chunk_store(r0, lds[1][0], lds[1][1], lds[1][2], bad);
    if (c + 3 < c1) pf_chunk_load(r0, A, lda, Wt, M, N, K, m0, n0, (c + 3) * PF_BK);
    vh_lds_sync();
    if (c + 1 >= c1) break;
    pf_chunk_mma(lds[1], wave, r, kq, acc, acl);
    if (c + 2 < c1) pf_chunk_store(r1, lds[0][0], lds[0][1], lds[0][2], bad);
    if (c + 4 < c1) pf_chunk_load(r1, A, lda, Wt, M, N, K, m0, n0, (c + 4) * PF_BK);
    vh_lds_sync();
  }
  if (bad) stc_u(err, VH_ERR_RANGE);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + 16 * j + r;
    if (n >= N) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = m0 + 16 * wave + 4 * (lane >> 4) + v;
      if (m >= M) continue;
      const float cv = fmaf(acl[j][v], 1.0f / VH_LO_SCALE, acc[j][v]);
      if (ksplit > 1)
        ws[((size_t)kp * M + m) * N + n] = cv;
      else
        pf_epi(mode, m, n, cv, bias, N, out, ldo, kc, vc, P, tp, layer, L, tmax);
    }
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

// ---------------------------------------------------------------- layer norm
// Y[i] = (X[r] - mean) / sqrt(var + 1e-5) * w + b for r = row0 + i * rstride
// (biased variance; mean and variance as sums of x / D and (x - mean)^2 / D,
// as gpt2.vst Q2 writes them): one block per output row, D <= 8 * 256,
// thread t holding the row's eight consecutive values 8t .. 8t + 7 (16-byte
// loads, so a wave's load is a whole kilobyte of the row), summed per thread,
// then over the block. With F set the row goes to F in fragment order (MT
// m-tiles: the thread writes its own piece) instead of Y. (Thread t on values
// t, t + 256, .., one 4-byte load each, measured slower: XL B=64 decode 4.06
// against 3.41 ms per step with the reduction below written that way.)
__device__ __forceinline__ void pf_ld8f(const float* p, float* v) {
  const vh_f32x4 a = *(const vh_f32x4*)p, b = *(const vh_f32x4*)(p + 4);
  v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3]; v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
}
__device__ __forceinline__ void pf_norm8_out(const float* v, const float* wv, const float* bv, bool in, int D, int i,
                                             float* __restrict__ Y, vh_half* __restrict__ F, int MT,
                                             unsigned* __restrict__ err, float* red) {
  const float fd = (float)D;
  float s = 0.0f;
  if (in)
#pragma unroll
    for (int j = 0; j < 8; ++j) s += v[j] / fd;
  const float mean = block_red_sum(s, red);
  float q = 0.0f;
  if (in)
#pragma unroll
    for (int j = 0; j < 8; ++j) q += (v[j] - mean) * (v[j] - mean) / fd;
  vh_lds_sync();
  const float sd = sqrtf(block_red_sum(q, red) + 0.00001f);
  if (!in) return;
  float y[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = (v[j] - mean) / sd * wv[j] + bv[j];
  const int k8 = 8 * threadIdx.x;
  if (F == nullptr) {
    float* yp = Y + (size_t)i * D + k8;
    *(vh_f32x4*)yp = vh_f32x4{y[0], y[1], y[2], y[3]};
    *(vh_f32x4*)(yp + 4) = vh_f32x4{y[4], y[5], y[6], y[7]};
    return;
  }
  bool bad = false;
  pf_frag_put8(F, MT, D / 32, i, k8, y, bad);
  if (bad) stc_u(err, VH_ERR_RANGE);
}

extern "C" __global__ __launch_bounds__(256) void pf_ln(const float* __restrict__ X, int row0, int rstride,
                                                         const vh_half* __restrict__ w, const vh_half* __restrict__ b,
                                                         float* __restrict__ Y, int D, vh_half* __restrict__ F, int MT,
                                                         unsigned* __restrict__ err) {
  __shared__ float red[VNWAVE];
  const int k8 = 8 * threadIdx.x;
  const bool in = k8 < D;
  float v[8] = {}, wv[8] = {}, bv[8] = {};
  if (in) {
    pf_ld8f(X + (size_t)(row0 + (size_t)blockIdx.x * rstride) * D + k8, v);
    unpack8(ld16(w + k8), wv);
    unpack8(ld16(b + k8), bv);
  }
  pf_norm8_out(v, wv, bv, in, D, blockIdx.x, Y, F, MT, err, red);
}

// pf_embed and the first layer's LayerNorm into fragment order (pf_ln) in one
// launch for a decode pass (one position per row): one block per row, the
// row kept in registers between the two.
extern "C" __global__ __launch_bounds__(256) void pf_embed_ln(const int* __restrict__ tok, const int* __restrict__ tp,
                                                               const vh_half* __restrict__ wte,
                                                               const vh_half* __restrict__ wpe, float* __restrict__ Z,
                                                               int D, int V, int npos, const vh_half* __restrict__ w,
                                                               const vh_half* __restrict__ b, vh_half* __restrict__ F,
                                                               int MT, unsigned* __restrict__ err) {
  __shared__ float red[VNWAVE];
  const int m = blockIdx.x, k8 = 8 * threadIdx.x;
  const bool in = k8 < D;
  int x = tok[m];
  x = x < 0 ? 0 : (x >= V ? V - 1 : x);
  int pos = *tp;
  pos = pos < 0 ? 0 : (pos >= npos ? npos - 1 : pos);
  float v[8] = {}, wv[8] = {}, bv[8] = {};
  if (in) {
    float a[8], c[8];
    unpack8(ld16(wte + (size_t)x * D + k8), a);
    unpack8(ld16(wpe + (size_t)pos * D + k8), c);
    unpack8(ld16(w + k8), wv);
    unpack8(ld16(b + k8), bv);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = a[j] + c[j];
    float* z = Z + (size_t)m * D + k8;
    *(vh_f32x4*)z = vh_f32x4{v[0], v[1], v[2], v[3]};
    *(vh_f32x4*)(z + 4) = vh_f32x4{v[4], v[5], v[6], v[7]};
  }
  pf_norm8_out(v, wv, bv, in, D, m, nullptr, F, MT, err, red);
}

// A split residual product's parts added in part order (pf_reduce, mode 1:
// Z[m, n] = (Z[m, n] + C) + bias[n]) and the LayerNorm that reads Z next (as
// pf_ln, into Y or F), in one launch: one block per row, the row kept in
// registers between the two.
extern "C" __global__ __launch_bounds__(256) void pf_reduce_ln(
    const float* __restrict__ ws, int ksplit, const vh_half* __restrict__ bias, int M, int D,
    float* __restrict__ Z, const vh_half* __restrict__ w, const vh_half* __restrict__ b, float* __restrict__ Y,
    vh_half* __restrict__ F, int MT, unsigned* __restrict__ err) {
  __shared__ float red[VNWAVE];
  const int m = blockIdx.x, k8 = 8 * threadIdx.x;
  const bool in = k8 < D;
  float v[8] = {}, zr[8] = {}, bn[8] = {}, wv[8] = {}, bv[8] = {};
  if (in) {
    pf_ld8f(ws + (size_t)m * D + k8, v);
    pf_ld8f(Z + (size_t)m * D + k8, zr);
    if (bias) unpack8(ld16(bias + k8), bn);
    unpack8(ld16(w + k8), wv);
    unpack8(ld16(b + k8), bv);
    for (int k0 = 1; k0 < ksplit; k0 += 4) {      // four parts' loads in flight, added in part order
      float p[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (k0 + u < ksplit) pf_ld8f(ws + ((size_t)(k0 + u) * M + m) * D + k8, p[u]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (k0 + u < ksplit)
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] += p[u][j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (zr[j] + v[j]) + bn[j];
    float* zp = Z + (size_t)m * D + k8;
    *(vh_f32x4*)zp = vh_f32x4{v[0], v[1], v[2], v[3]};
    *(vh_f32x4*)(zp + 4) = vh_f32x4{v[4], v[5], v[6], v[7]};
  }
  pf_norm8_out(v, wv, bv, in, D, m, Y, F, MT, err, red);
}

// ---------------------------------------------------------------- decode products
// C = A W over K for M <= 16 MT rows, both operands in fragment order (above):
// the weights streamed from memory straight into the matrix cores' registers,
// the activations read as they are (hi and lo planes, each multiplied into
// its own accumulator and combined at the end). A block is PF_MW waves on the
// same MN n-tiles of 16 columns, MN = 1 up to 32 rows and 2 at 64 rows (with
// MN = 2 throughout, same box: GPT-2 small at 32 rows 0.585 -> 0.601 ms per
// step, medium at 16 rows 0.969 -> 1.058, XL at 64 rows even; with MN = 1 at
// 64 rows XL 3.02 -> 3.79, the activation rows re-read by twice the blocks);
// block vb takes n-tiles MN (vb / ks) .. + MN and fold part vb % ks of ks,
// and its waves split that part's k-steps into PF_MW consecutive runs. A
// wave with at most PF_WFIRST k-steps issues all its
// weight fragments at once, then the activation fragments one k-step ahead
// of the one it multiplies (XL B=64 decode 3.35 -> 3.10 ms per step against
// both one k-step ahead; activations two ahead 3.15); a longer run keeps the
// next k-step's weights and activations in flight. The waves' partial tiles
// are added in LDS in wave order. Then either the part is stored (ks > 1:
// ws[part][m][n], added by pf_reduce / pf_reduce_ln / pf_reduce_frag), or the
// epilogue of `mode` is applied: 0, 1 and 3 as pf_epi (one position per row);
// 2 (GELU) writes the result in fragment order into F, as the activation of
// the next product (N / 32 k-steps).
#define PF_MW 8
#define PF_WFIRST 8     // k-steps of a wave up to which all its weight fragments are loaded first

// pf_epi for eight consecutive columns n .. n + 7 of row m (one position per
// row), modes 1 (residual) and 3 (qkv: queries, or eight values of a key /
// value cache row as one 16-byte store); the same arithmetic per value.
__device__ __forceinline__ void pf_epi8(int mode, int m, int n, float* v, const float* bn, const float* z, int pos,
                                        int N, float* __restrict__ out, int ldo, vh_half* __restrict__ kc,
                                        vh_half* __restrict__ vc, int layer, int L, int tmax) {
  if (mode == 1) {
    float* o = out + (size_t)m * ldo + n;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (z[j] + v[j]) + bn[j];
    *(vh_f32x4*)o = vh_f32x4{v[0], v[1], v[2], v[3]};
    *(vh_f32x4*)(o + 4) = vh_f32x4{v[4], v[5], v[6], v[7]};
    return;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = v[j] + bn[j];
  const int D = N / 3;
  if (n < D) {
    float* o = out + (size_t)m * ldo + n;
    *(vh_f32x4*)o = vh_f32x4{v[0], v[1], v[2], v[3]};
    *(vh_f32x4*)(o + 4) = vh_f32x4{v[4], v[5], v[6], v[7]};
    return;
  }
  if (pos < 0 || pos >= tmax) return;
  unsigned short h[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = f2h(v[j]);
  const size_t at = ((size_t)(m * L + layer) * tmax + pos) * D + (n % D);
  *(vh_u32x4*)((n < 2 * D ? kc : vc) + at) =
      vh_u32x4{h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16), h[4] | ((unsigned)h[5] << 16),
               h[6] | ((unsigned)h[7] << 16)};
}
template <int MT, int MN, bool WNT>
__device__ __forceinline__ void pf_mgemm_body(
    int vb, const vh_u32x4* __restrict__ Af, const vh_u32x4* __restrict__ Wf, int KT, int NT, int ks,
    const vh_half* __restrict__ bias, int M, int N, int mode, float* __restrict__ out, int ldo,
    vh_half* __restrict__ kc, vh_half* __restrict__ vc, const int* __restrict__ tp, int layer, int L, int tmax,
    float* __restrict__ ws, vh_half* __restrict__ F, unsigned* __restrict__ err) {
  __shared__ __attribute__((aligned(16))) vh_f32x4 red[PF_MW][MN * MT * 64];
  __shared__ __attribute__((aligned(16))) float tile[16 * MT][16 * MN + 4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int part = vb % ks, nt0 = (vb / ks) * MN;
  const int ka = part * KT / ks, kb = (part + 1) * KT / ks;
  const int k0 = ka + (kb - ka) * wave / PF_MW, k1 = ka + (kb - ka) * (wave + 1) / PF_MW;
  vh_f32x4 acc[MN][MT], acl[MN][MT];
#pragma unroll
  for (int t = 0; t < MN; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = acl[t][mt] = vh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const size_t plane = (size_t)MT * KT * 64;
  // the epilogue's operands of this thread's item (a thread has at most one:
  // 16 MT x 2 MN <= PF_MW x 64), loaded before the products so that their
  // latency is not added at the end: the bias, the residual row piece, the
  // sequence position of the cache rows
  const int ei = threadIdx.x, em = ei / (2 * MN), ec8 = 8 * (ei % (2 * MN)), en = 16 * nt0 + ec8;
  const bool eok = ks == 1 && ei < 16 * MT * 2 * MN && em < M && en < N;
  float eb[8] = {}, ez[8] = {};
  int epos = 0;
  // the GELU product adds the bias and applies GELU where the waves' sums are
  // added (every thread has at most one item there: MN MT 64 <= PF_MW 64),
  // so that all threads share that work; this thread's item's column bias:
  const bool gelu_red = ks == 1 && mode == 2;
  const int rn = 16 * (nt0 + (threadIdx.x >> 6) / MT) + (threadIdx.x & 15);
  const float rb = gelu_red && bias != nullptr && threadIdx.x < MN * MT * 64 && rn < N ? h2f(bias[rn]) : 0.0f;
  if (eok) {
    if (bias && mode != 2) unpack8(ld16(bias + en), eb);
    if (mode == 1) pf_ld8f(out + (size_t)em * ldo + en, ez);
    if (mode == 3) epos = *tp;
  }
  // weight fragments: nontemporal (WNT) where the model's weights cannot stay
  // in the memory-side cache between steps (the host picks the kernel)
  auto wld = [&](size_t i) {
    if constexpr (WNT)
      return __builtin_nontemporal_load(Wf + i);
    else
      return Wf[i];
  };
  vh_u32x4 wa[MN], aa[2][MT], wb[MN], ab[2][MT];
  auto load = [&](vh_u32x4 (&w)[MN], vh_u32x4 (&a)[2][MT], int k) {
    const bool in = k < k1;
#pragma unroll
    for (int t = 0; t < MN; ++t)
      w[t] = in && nt0 + t < NT ? wld(((size_t)(nt0 + t) * KT + k) * 64 + lane) : vh_u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        a[p][mt] = in ? Af[p * plane + ((size_t)mt * KT + k) * 64 + lane] : vh_u32x4{0u, 0u, 0u, 0u};
  };
  auto mma = [&](const vh_u32x4 (&w)[MN], const vh_u32x4 (&a)[2][MT]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < MN; ++t) {
        acc[t][mt] = vh_mfma(a[0][mt], w[t], acc[t][mt]);
        acl[t][mt] = vh_mfma(a[1][mt], w[t], acl[t][mt]);
      }
  };
  if (k1 - k0 <= PF_WFIRST) {
    // all of the wave's weight fragments first (so they are in flight at once),
    // then the activation fragments one k-step ahead
    vh_u32x4 wall[PF_WFIRST][MN];
#pragma unroll
    for (int j = 0; j < PF_WFIRST; ++j)
#pragma unroll
      for (int t = 0; t < MN; ++t)
        wall[j][t] = k0 + j < k1 && nt0 + t < NT ? wld(((size_t)(nt0 + t) * KT + k0 + j) * 64 + lane)
                                                 : vh_u32x4{0u, 0u, 0u, 0u};
    auto loada = [&](vh_u32x4 (&a)[2][MT], int k) {
      const bool in = k < k1;
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          a[p][mt] = in ? Af[p * plane + ((size_t)mt * KT + k) * 64 + lane] : vh_u32x4{0u, 0u, 0u, 0u};
    };
    loada(aa, k0);
#pragma unroll
    for (int j = 0; j < PF_WFIRST; j += 2) {
      if (k0 + j < k1) {
        loada(ab, k0 + j + 1);
        mma(wall[j], aa);
      }
      if (k0 + j + 1 < k1) {
        loada(aa, k0 + j + 2);
        mma(wall[j + 1], ab);
      }
    }
  } else {
    load(wa, aa, k0);
    for (int k = k0; k < k1; k += 2) {
      load(wb, ab, k + 1);
      mma(wa, aa);
      if (k + 1 >= k1) break;
      load(wa, aa, k + 2);
      mma(wb, ab);
    }
  }
#pragma unroll
  for (int t = 0; t < MN; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const vh_f32x4 h = acc[t][mt], l = acl[t][mt];
      red[wave][(t * MT + mt) * 64 + lane] =
          vh_f32x4{vh_hilo(h[0], l[0]), vh_hilo(h[1], l[1]), vh_hilo(h[2], l[2]), vh_hilo(h[3], l[3])};
    }
  __syncthreads();
  for (int i = threadIdx.x; i < MN * MT * 64; i += PF_MW * 64) {
    vh_f32x4 s = red[0][i];
#pragma unroll
    for (int w = 1; w < PF_MW; ++w) {
      const vh_f32x4 o = red[w][i];
      s = vh_f32x4{s[0] + o[0], s[1] + o[1], s[2] + o[2], s[3] + o[3]};
    }
    const int l = i & 63, tm = i >> 6, mt = tm % MT, t = tm / MT;
    if (gelu_red)
#pragma unroll
      for (int v = 0; v < 4; ++v) s[v] = pf_gelu(s[v] + rb);
#pragma unroll
    for (int v = 0; v < 4; ++v) tile[16 * mt + 4 * (l >> 4) + v][16 * t + (l & 15)] = s[v];
  }
  __syncthreads();
  const int n0 = 16 * nt0;
  if (ks == 1 && mode == 2) {
    bool bad = false;
    for (int e = threadIdx.x; e < 16 * MT * 2 * MN; e += PF_MW * 64) {
      const int m = e / (2 * MN), c8 = 8 * (e % (2 * MN));
      if (m >= M || n0 + c8 >= N) continue;
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = tile[m][c8 + j];     // bias and GELU applied above
      pf_frag_put8(F, MT, N / 32, m, n0 + c8, v, bad);
    }
    if (bad) stc_u(err, VH_ERR_RANGE);
    return;
  }
  if (ks > 1 || mode == 1 || mode == 3) {   // eight consecutive columns per thread, 16-byte stores
    for (int e = threadIdx.x; e < 16 * MT * 2 * MN; e += PF_MW * 64) {
      const int m = e / (2 * MN), c8 = 8 * (e % (2 * MN)), n = n0 + c8;
      if (m >= M || n >= N) continue;
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = tile[m][c8 + j];
      if (ks > 1) {
        float* p = ws + ((size_t)part * M + m) * N + n;
        *(vh_f32x4*)p = vh_f32x4{v[0], v[1], v[2], v[3]};
        *(vh_f32x4*)(p + 4) = vh_f32x4{v[4], v[5], v[6], v[7]};
      } else {
        pf_epi8(mode, m, n, v, eb, ez, epos, N, out, ldo, kc, vc, layer, L, tmax);     // (e is this thread's item)
      }
    }
    return;
  }
  for (int e = threadIdx.x; e < 16 * MT * 16 * MN; e += PF_MW * 64) {
    const int m = e / (16 * MN), c = e % (16 * MN), n = n0 + c;
    if (m >= M || n >= N) continue;
    pf_epi(mode, m, n, tile[m][c], bias, N, out, ldo, kc, vc, 1, tp, layer, L, tmax);
  }
}

#define PF_MGEMM(name, MT, MN, WNT)                                                                                     \
  extern "C" __global__ __launch_bounds__(PF_MW * 64) void name(                                                  \
      const vh_u32x4* __restrict__ Af, const vh_u32x4* __restrict__ Wf, int KT, int NT, int ks,                    \
      const vh_half* __restrict__ bias, int M, int N, int mode, float* __restrict__ out, int ldo,                 \
      vh_half* __restrict__ kc, vh_half* __restrict__ vc, const int* __restrict__ tp, int layer, int L, int tmax, \
      float* __restrict__ ws, vh_half* __restrict__ F, unsigned* __restrict__ err) {                              \
    pf_mgemm_body<MT, MN, WNT>(blockIdx.x, Af, Wf, KT, NT, ks, bias, M, N, mode, out, ldo, kc, vc, tp, layer, L,    \
                               tmax, ws, F, err);                                                                 \
  }
PF_MGEMM(pf_mgemm1, 1, 1, false)
PF_MGEMM(pf_mgemm2, 2, 1, false)
PF_MGEMM(pf_mgemm4, 4, 2, false)
PF_MGEMM(pf_mgemm1n, 1, 1, true)
PF_MGEMM(pf_mgemm2n, 2, 1, true)
PF_MGEMM(pf_mgemm4n, 4, 2, true)

// The output head (a plain product with many columns: out[m, n] = C, no
// bias): block b's wave w makes n-tiles 2 (PF_MW b + w) and the next one
// over the whole fold, weights and activations one k-step ahead. The block's
// waves read the same activation fragments at about the same time, so they
// come from the CU's L1 after the first wave: the activations cross from L2
// once per block, not once per pair of n-tiles as in pf_mgemm*. The sums go
// straight from the accumulators to out (lane l: rows 4 (l / 16) .. +4 of
// column l % 16).
template <int MT>
__device__ __forceinline__ void pf_mhead_body(const vh_u32x4* __restrict__ Af, const vh_u32x4* __restrict__ Wf, int KT,
                                              int NT, int M, int N, float* __restrict__ out, int ldo) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nt0 = 2 * (PF_MW * (int)blockIdx.x + wave);
  if (nt0 >= NT) return;
  vh_f32x4 acc[2][MT], acl[2][MT];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = acl[t][mt] = vh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const size_t plane = (size_t)MT * KT * 64;
  vh_u32x4 wa[2], aa[2][MT], wb[2], ab[2][MT];
  auto load = [&](vh_u32x4 (&w)[2], vh_u32x4 (&a)[2][MT], int k) {
    const bool in = k < KT;
#pragma unroll
    for (int t = 0; t < 2; ++t)
      w[t] = in && nt0 + t < NT ? Wf[((size_t)(nt0 + t) * KT + k) * 64 + lane] : vh_u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        a[p][mt] = in ? Af[p * plane + ((size_t)mt * KT + k) * 64 + lane] : vh_u32x4{0u, 0u, 0u, 0u};
  };
  auto mma = [&](const vh_u32x4 (&w)[2], const vh_u32x4 (&a)[2][MT]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        acc[t][mt] = vh_mfma(a[0][mt], w[t], acc[t][mt]);
        acl[t][mt] = vh_mfma(a[1][mt], w[t], acl[t][mt]);
      }
  };
  load(wa, aa, 0);
  for (int k = 0; k < KT; k += 2) {
    load(wb, ab, k + 1);
    mma(wa, aa);
    if (k + 1 >= KT) break;
    load(wa, aa, k + 2);
    mma(wb, ab);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int n = 16 * (nt0 + t) + (lane & 15);
    if (nt0 + t >= NT || n >= N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = 16 * mt + 4 * (lane >> 4) + v;
        if (m < M) out[(size_t)m * ldo + n] = vh_hilo(acc[t][mt][v], acl[t][mt][v]);
      }
  }
}
#define PF_MHEAD(name, MT)                                                                                         \
  extern "C" __global__ __launch_bounds__(PF_MW * 64) void name(const vh_u32x4* __restrict__ Af,                 \
                                                                const vh_u32x4* __restrict__ Wf, int KT, int NT,  \
                                                                int M, int N, float* __restrict__ out, int ldo) {  \
    pf_mhead_body<MT>(Af, Wf, KT, NT, M, N, out, ldo);                                                           \
  }
PF_MHEAD(pf_mhead1, 1)
PF_MHEAD(pf_mhead2, 2)
PF_MHEAD(pf_mhead4, 4)

// The parts of a split GELU product (ws[part][m][n], part order) with the
// bias and GELU, written in fragment order into F like pf_mgemm's mode 2: one
// thread per eight consecutive columns of a row.
extern "C" __global__ __launch_bounds__(256) void pf_reduce_frag(const float* __restrict__ ws, int ksplit,
                                                                  const vh_half* __restrict__ bias, int M, int N,
                                                                  vh_half* __restrict__ F, int MT,
                                                                  unsigned* __restrict__ err) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= M * (N / 8)) return;
  const int m = e / (N / 8), n8 = 8 * (e % (N / 8));
  float v[8];
  const float* p = ws + (size_t)m * N + n8;
  pf_ld8f(p, v);
  for (int k = 1; k < ksplit; ++k) {
    float q[8];
    pf_ld8f(p + (size_t)k * M * N, q);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] += q[j];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = pf_gelu(v[j] + h2f(bias[n8 + j]));
  bool bad = false;
  pf_frag_put8(F, MT, N / 32, m, n8, v, bad);
  if (bad) stc_u(err, VH_ERR_RANGE);
}

// ---------------------------------------------------------------- attention
// One wave per (row m, head h): scores of the query against cache positions
// 0 .. t0 + p (gpt2.vst Q5: dot over e, divided by 8; eight lanes per
// position, each a 16-byte piece of the key row, the partial dots added
// across them),
// the max-subtracted softmax (Q6), and the weighted values (Q7: eight lanes
// per position, 8 dims each), read from the fp16 cache the qkv product just
// wrote. O[m, h * 64 + e] receives the head's output.
// `ws` holds each wave's scores, then weights, for up to PF_TMAX positions.
extern "C" __global__ __launch_bounds__(256) void pf_attn(const float* __restrict__ Q, const vh_half* __restrict__ kc,
                                                           const vh_half* __restrict__ vc, float* __restrict__ O,
                                                           int M, int P, const int* __restrict__ tp, int layer,
                                                           int L, int tmax, int H) {
  __shared__ float ws[VNWAVE][PF_TMAX];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int item = blockIdx.x * VNWAVE + wave;
  const bool live = item < M * H;
  const int m = live ? item / H : 0, h = live ? item % H : 0;
  const int D = H * PF_E;
  const int b = m / P, at = *tp + m % P;
  const int pos = at < tmax ? at : tmax - 1;
  const size_t base = (size_t)(b * L + layer) * tmax * D + (size_t)h * PF_E;
  // scores: eight lanes per position (lane 8g + c holds dims 8c .. 8c + 7,
  // one 16-byte load), positions g, g + 8, .. of the wave's 8 lane groups,
  // four in flight per lane; the eight partial dots added across the group
  const int g = lane >> 3, c8 = lane & 7;
  float qv[8];
  {
    const float* qp = Q + (size_t)m * D + h * PF_E + 8 * c8;
    const vh_f32x4 q0 = live ? *(const vh_f32x4*)qp : vh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const vh_f32x4 q1 = live ? *(const vh_f32x4*)(qp + 4) : vh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    qv[0] = q0[0]; qv[1] = q0[1]; qv[2] = q0[2]; qv[3] = q0[3];
    qv[4] = q1[0]; qv[5] = q1[1]; qv[6] = q1[2]; qv[7] = q1[3];
  }
  float mx = -INFINITY;
  if (live) {
    for (int s0 = g; s0 <= pos; s0 += 8 * 4) {
      vh_u32x4 kr[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int s = s0 + 8 * u;
        kr[u] = s <= pos ? ld16(kc + base + (size_t)s * D + 8 * c8) : vh_u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float kv[8];
        unpack8(kr[u], kv);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = fmaf(qv[j], kv[j], acc);
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        acc += __shfl_xor(acc, 4, 64);
        const int s = s0 + 8 * u;
        if (s <= pos) {
          const float sc = acc * 0.125f;      // / 8, exact
          if (c8 == 0) ws[wave][s] = sc;
          mx = fmaxf(mx, sc);
        }
      }
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
    // lane 8a + b sums positions s = a (mod 8) over dims 8b..8b+7 (one 16-byte
    // load of a row per position), four positions of its residue in flight;
    // then the eight residues are added across lanes
    const int a = lane >> 3, b = lane & 7;
    float o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 <= pos; s0 += 32) {
      vh_u32x4 vr[4];
      float wv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int s = s0 + 8 * u + a;
        const bool in = s <= pos;
        vr[u] = in ? ld16(vc + base + (size_t)s * D + 8 * b) : vh_u32x4{0u, 0u, 0u, 0u};
        wv[u] = in ? ws[wave][s] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float v[8];
        unpack8(vr[u], v);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = fmaf(wv[u], v[j], o[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o[j] += __shfl_xor(o[j], 8, 64);
      o[j] += __shfl_xor(o[j], 16, 64);
      o[j] += __shfl_xor(o[j], 32, 64);
    }
    if (a == 0) {
      float* dst = O + (size_t)m * D + h * PF_E + 8 * b;
      *(vh_f32x4*)dst = vh_f32x4{o[0], o[1], o[2], o[3]};
      *(vh_f32x4*)(dst + 4) = vh_f32x4{o[4], o[5], o[6], o[7]};
    }
  }
}

// One position per row (a decode step): one block per (row m, head h), every
// thread of the block on the positions 0 .. t0, so that a step's cache rows
// are read with a block's worth of loads in flight instead of a wave's. Each
// score is read by eight lanes, one 16-byte piece of the position's key row
// each (so a wave's load covers eight whole rows), the eight partial dots
// added across the lanes, / 8; the max-subtracted softmax (block-wide maximum
// and sum); the weighted values with wave w, lane 8a + b on positions
// s = 8w + a (mod 32), dims 8b..8b+7, the four waves' partial outputs added
// in order through LDS. (Keys read a row per lane, eight 16-byte loads of it,
// measured slower: XL B=64 decode 4.32 against 4.06 ms per step.) The cache
// rows are loaded nontemporal here and in pf_attn1s: a step reads each once,
// and with the default policy they displaced the products' weights from the
// caches (same box: GPT-2 small at 32 rows 0.586 -> 0.550 ms per step, the
// attention launch 19.3 -> 17.8 us; XL at 64 rows 3.023 -> 3.000).
extern "C" __global__ __launch_bounds__(256) void pf_attn1(const float* __restrict__ Q, const vh_half* __restrict__ kc,
                                                            const vh_half* __restrict__ vc, float* __restrict__ O,
                                                            const int* __restrict__ tp, int layer, int L, int tmax,
                                                            int H, vh_half* __restrict__ F, int MT,
                                                            unsigned* __restrict__ err) {
  __shared__ float qs[PF_E];
  __shared__ float ws[PF_TMAX];
  __shared__ float red[VNWAVE];
  __shared__ float part[VNWAVE][PF_E];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = blockIdx.x / H, h = blockIdx.x % H;      // grid: rows * H blocks exactly
  const int D = H * PF_E;
  const size_t base = (size_t)(m * L + layer) * tmax * D + (size_t)h * PF_E;
  // scores: eight lanes per position (lane 8g + b holds dims 8b .. 8b + 7, one
  // 16-byte load), positions g, g + 32, .. of the block's 32 lane groups, four
  // in flight per lane; the eight partial dots added across the group. The
  // query and the first batch (positions below 128, clamped into the cache) are
  // loaded before the position is read, so that their round trips overlap;
  // the batch's positions beyond the step's are loaded but not used.
  const int g = tid >> 3, b8 = tid & 7;
  float qv[8];
  {
    const float* qp = Q + (size_t)m * D + h * PF_E + 8 * b8;
    const vh_f32x4 q0 = *(const vh_f32x4*)qp, q1 = *(const vh_f32x4*)(qp + 4);
    qv[0] = q0[0]; qv[1] = q0[1]; qv[2] = q0[2]; qv[3] = q0[3];
    qv[4] = q1[0]; qv[5] = q1[1]; qv[6] = q1[2]; qv[7] = q1[3];
  }
  vh_u32x4 kr[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int s = g + 32 * u < tmax ? g + 32 * u : tmax - 1;     // clamped: loads without a branch
    kr[u] = ld16_nt(kc + base + (size_t)s * D + 8 * b8);
  }
  __builtin_amdgcn_sched_barrier(0);    // the loads above issued before the position is waited for
  const int at = *tp;
  const int pos = at < tmax ? at : tmax - 1;
  float mx = -INFINITY;
  int s0 = g;
  do {                                  // the first batch even where g > pos (then none of it is used)
    if (s0 != g) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int s = s0 + 32 * u;
        kr[u] = s <= pos ? ld16_nt(kc + base + (size_t)s * D + 8 * b8) : vh_u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float kv[8];
      unpack8(kr[u], kv);
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = fmaf(qv[j], kv[j], acc);
      acc += __shfl_xor(acc, 1, 64);
      acc += __shfl_xor(acc, 2, 64);
      acc += __shfl_xor(acc, 4, 64);
      const int s = s0 + 32 * u;
      if (s <= pos) {
        const float sc = acc * 0.125f;      // / 8, exact
        if (b8 == 0) ws[s] = sc;
        mx = fmaxf(mx, sc);
      }
    }
    s0 += 32 * 4;
  } while (s0 <= pos);
  __syncthreads();                      // ws written by the groups' first lanes, read by all below
  mx = wave_red_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < VNWAVE; ++w) mx = fmaxf(mx, red[w]);
  __syncthreads();                      // red is reused for the sum
  float sum = 0.0f;
  for (int s = tid; s <= pos; s += VBLOCK) {
    const float ex = expf(ws[s] - mx);
    ws[s] = ex;
    sum += ex;
  }
  sum = wave_red_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  sum = red[0];
#pragma unroll
  for (int w = 1; w < VNWAVE; ++w) sum += red[w];
  for (int s = tid; s <= pos; s += VBLOCK) ws[s] = ws[s] / sum;
  __syncthreads();
  const int a = lane >> 3, b = lane & 7;
  float o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 8 * wave; s0 <= pos; s0 += 32 * 4) {
    vh_u32x4 vr[4];
    float wv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = s0 + 32 * u + a;
      const bool in = s <= pos;
      vr[u] = in ? ld16_nt(vc + base + (size_t)s * D + 8 * b) : vh_u32x4{0u, 0u, 0u, 0u};
      wv[u] = in ? ws[s] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float v[8];
      unpack8(vr[u], v);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = fmaf(wv[u], v[j], o[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    o[j] += __shfl_xor(o[j], 8, 64);
    o[j] += __shfl_xor(o[j], 16, 64);
    o[j] += __shfl_xor(o[j], 32, 64);
  }
  if (a == 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) part[wave][8 * b + j] = o[j];
  }
  __syncthreads();
  if (tid < PF_E) {
    float r = part[0][tid];
#pragma unroll
    for (int w = 1; w < VNWAVE; ++w) r += part[w][tid];
    if (F == nullptr)
      O[(size_t)m * D + h * PF_E + tid] = r;
    else
      qs[tid] = r;
  }
  if (F != nullptr) {       // the head's 64 outputs in fragment order, eight per thread
    __syncthreads();
    bool bad = false;
    if (tid < PF_E / 8) pf_frag_put8(F, MT, D / 32, m, h * PF_E + 8 * tid, qs + 8 * tid, bad);
    if (bad) stc_u(err, VH_ERR_RANGE);
  }
}

// pf_attn1 in one pass over the cache (a running softmax): lane group g
// (eight lanes, one 16-byte piece of a row each) takes positions g, g + 32, ..
// and loads each position's key and value pieces together, four positions a
// batch. Per batch the group's running maximum m becomes max(m, its scores),
// its sum l and weighted values (eight dims per lane) are rescaled by
// exp(m_old - m) and the batch's exp(score - m) added. The 32 groups are then
// combined in group order, each rescaled by exp(m_g - max_g m_g): the output is
// the sum of the weighted values over the sum of the l's. One round trip to
// the cache per batch instead of one for the keys and one for the values:
// faster where there are few (row, head) blocks (GPT-2 small, 32 rows, 1024
// positions: 0.666 -> 0.637 ms per step), not with many (XL, 64 rows x 25
// heads: 3.110 -> 3.128), so the decode pass takes it up to
// ATTN_ONE_PASS_BLOCKS blocks. The first batch (positions below 128, clamped into
// the cache) is loaded before the position is read, so that its round trip
// overlaps that read and the query's; its positions beyond the step's are
// loaded but not used.
extern "C" __global__ __launch_bounds__(256) void pf_attn1s(const float* __restrict__ Q, const vh_half* __restrict__ kc,
                                                             const vh_half* __restrict__ vc, float* __restrict__ O,
                                                             const int* __restrict__ tp, int layer, int L, int tmax,
                                                             int H, vh_half* __restrict__ F, int MT,
                                                             unsigned* __restrict__ err) {
  __shared__ float qs[PF_E];
  __shared__ float gm[32], gl[32], gf[32];
  __shared__ float part[32][PF_E];
  const int tid = threadIdx.x;
  const int m = blockIdx.x / H, h = blockIdx.x % H;      // grid: rows * H blocks exactly
  const int D = H * PF_E;
  const size_t base = (size_t)(m * L + layer) * tmax * D + (size_t)h * PF_E;
  const int g = tid >> 3, b8 = tid & 7;
  float qv[8];
  {
    const float* qp = Q + (size_t)m * D + h * PF_E + 8 * b8;
    const vh_f32x4 q0 = *(const vh_f32x4*)qp, q1 = *(const vh_f32x4*)(qp + 4);
    qv[0] = q0[0]; qv[1] = q0[1]; qv[2] = q0[2]; qv[3] = q0[3];
    qv[4] = q1[0]; qv[5] = q1[1]; qv[6] = q1[2]; qv[7] = q1[3];
  }
  vh_u32x4 kr[4], vr[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int s = g + 32 * u < tmax ? g + 32 * u : tmax - 1;     // clamped: loads without a branch
    const size_t at8 = base + (size_t)s * D + 8 * b8;
    kr[u] = ld16_nt(kc + at8);
    vr[u] = ld16_nt(vc + at8);
  }
  __builtin_amdgcn_sched_barrier(0);    // the loads above issued before the position is waited for
  const int at = *tp;
  const int pos = at < tmax ? at : tmax - 1;
  float mx = -INFINITY, sm = 0.0f, o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  int s0 = g;
  do {                                      // the first batch even where g > pos (then none of it is used)
    if (s0 != g) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int s = s0 + 32 * u;
        const size_t at8 = base + (size_t)s * D + 8 * b8;
        kr[u] = s <= pos ? ld16_nt(kc + at8) : vh_u32x4{0u, 0u, 0u, 0u};
        vr[u] = s <= pos ? ld16_nt(vc + at8) : vh_u32x4{0u, 0u, 0u, 0u};
      }
    }
    float sc[4];
    float bm = mx;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float kv[8];
      unpack8(kr[u], kv);
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = fmaf(qv[j], kv[j], acc);
      acc += __shfl_xor(acc, 1, 64);
      acc += __shfl_xor(acc, 2, 64);
      acc += __shfl_xor(acc, 4, 64);
      sc[u] = acc * 0.125f;                 // / 8, exact
      if (s0 + 32 * u <= pos) bm = fmaxf(bm, sc[u]);
    }
    const float c = bm == -INFINITY ? 0.0f : expf(mx - bm);   // 0 while mx is -inf, or no position yet
    sm *= c;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] *= c;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (s0 + 32 * u > pos) continue;
      const float p = expf(sc[u] - bm);
      float v[8];
      unpack8(vr[u], v);
      sm += p;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = fmaf(p, v[j], o[j]);
    }
    mx = bm;
    s0 += 32 * 4;
  } while (s0 <= pos);
  if (b8 == 0) {
    gm[g] = mx;
    gl[g] = sm;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) part[g][8 * b8 + j] = o[j];
  __syncthreads();
  if (tid < 32) {             // each group's scale (0 for a group with no position)
    float M = gm[0];
    for (int k = 1; k < 32; ++k) M = fmaxf(M, gm[k]);
    gf[tid] = gm[tid] == -INFINITY ? 0.0f : expf(gm[tid] - M);
  }
  __syncthreads();
  if (tid < PF_E) {
    float l = 0.0f, r = 0.0f;
    for (int k = 0; k < 32; ++k) {
      l = fmaf(gl[k], gf[k], l);
      r = fmaf(part[k][tid], gf[k], r);
    }
    r = r / l;
    if (F == nullptr)
      O[(size_t)m * D + h * PF_E + tid] = r;
    else
      qs[tid] = r;
  }
  if (F != nullptr) {       // the head's 64 outputs in fragment order, eight per thread
    __syncthreads();
    bool bad = false;
    if (tid < PF_E / 8) pf_frag_put8(F, MT, D / 32, m, h * PF_E + 8 * tid, qs + 8 * tid, bad);
    if (bad) stc_u(err, VH_ERR_RANGE);
  }
}

// ---------------------------------------------------------------- argmax
// Per row of logits [B, V]: the largest value, a tie to the lowest id
// (gpt2.vst Q10), in two launches so that a row is read by S blocks at once.
// pf_argmax_part: block b * S + s takes chunk s of row b and writes its pair
// (value, id) to pv / pi. pf_argmax: one block per row combines the S pairs
// (the rule picks the same pair in any order), writes the token into x (the
// next step's input) and, as a float, into `next`; block 0 advances the
// position counter by P.
extern "C" __global__ __launch_bounds__(256) void pf_argmax_part(const float* __restrict__ logit, int V, int S,
                                                                  float* __restrict__ pv, int* __restrict__ pi) {
  __shared__ float rv[VNWAVE];
  __shared__ int ri[VNWAVE];
  const int b = blockIdx.x / S, s = blockIdx.x % S;
  const int chunk = (V + S - 1) / S;
  const int n0 = s * chunk, n1 = min(V, n0 + chunk);
  const float* lg = logit + (size_t)b * V;
  float best = -INFINITY;
  int id = V;
#pragma unroll 4
  for (int n = n0 + (int)threadIdx.x; n < n1; n += VBLOCK) argmax_pair(best, id, lg[n], n);
  block_argmax(best, id, rv, ri);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = best;
    pi[blockIdx.x] = id;
  }
}

extern "C" __global__ __launch_bounds__(256) void pf_argmax(const float* __restrict__ pv, const int* __restrict__ pi,
                                                             int S, int* __restrict__ x, float* __restrict__ next,
                                                             int* __restrict__ tp, int P) {
  __shared__ float rv[VNWAVE];
  __shared__ int ri[VNWAVE];
  float best = -INFINITY;
  int id = 0x7fffffff;
  for (int k = threadIdx.x; k < S; k += VBLOCK) argmax_pair(best, id, pv[blockIdx.x * S + k], pi[blockIdx.x * S + k]);
  block_argmax(best, id, rv, ri);
  if (threadIdx.x == 0) {
    x[blockIdx.x] = id;
    next[blockIdx.x] = (float)id;
    if (blockIdx.x == 0) *tp += P;     // the last kernel of a pass: advance the position
  }
}
