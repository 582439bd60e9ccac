/*
 * cmoe.c - C restatement of the MoE decode layer (bf16 rounding points).
 *
 * TEST INFRASTRUCTURE ONLY: the timed CPU baseline of bench.py and a checker
 * in tests/.  Same semantics as oracle/moe_oracle.py, mode "bf16", path
 * "decode" (the reference's _moe_call at threshold 1.0 with the fused combine,
 * models/flashnext/adaptive_topk.py:54-293 and metal_runtime.py:231-336),
 * with float32 accumulation as MLX's CPU and Metal kernels use:
 *   logits  = bf16(x . Wr^T (+ bias));  gates = bf16(softmax)  (fp32)
 *   top-k by (gate desc, index asc);    scores = bf16(g / bf16(sum g))
 *   projection row = sum_g s*sum(x*q) + b*sum(x)   (Q4/G32, MLX nibble order)
 *   act = bf16 op-by-op SwiGLU;  y = bf16(bf16(sum_j bf16(d_j)*s_j) + shared_y)
 * Parallel over output rows with OpenMP.  Experts are read from fixed-stride
 * records (the expert pool layout) through an expert -> record table.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct CmoeQ4 {
  const uint32_t* w; /* [out, in/8] */
  const uint16_t* s; /* [out, in/32] */
  const uint16_t* b;
} CmoeQ4;

typedef struct CmoeLayer {
  int hidden, inter, experts, top_k, shared_inter;
  const uint16_t* router;      /* [E, H] bf16 */
  const float* router_bias;    /* [E] or NULL */
  const uint8_t* records;      /* expert records */
  uint64_t record_stride;
  uint64_t offsets[9];         /* gate w,s,b  up w,s,b  down w,s,b */
  const int32_t* record_of;    /* [E] expert -> record index, or NULL (identity) */
  CmoeQ4 sgate, sup, sdown, segate; /* shared expert and its H -> 1 gate */
} CmoeLayer;

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float r16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

static float exp32(float v) { return (float)exp((double)v); }

static float sigmoid_bf16(float g) {
  float mag = fabsf(g);
  float e = r16(exp32(mag));
  float den = r16(1.0f + e);
  float small = r16(1.0f / den);
  return g < 0.0f ? small : r16(1.0f - small);
}

static float swiglu_bf16(float g, float u) {
  float s = r16(g * sigmoid_bf16(g));
  return r16(s * u);
}

/* one Q4/G32 row: w [in/8] words, s/b [in/32] */
static float q4_row(const float* x, const uint32_t* w, const uint16_t* s, const uint16_t* b, int in) {
  float acc = 0.0f;
  const int groups = in / 32;
  for (int g = 0; g < groups; ++g) {
    float qsum = 0.0f, xsum = 0.0f;
    const uint32_t* wg = w + g * 4;
    const float* xg = x + g * 32;
    for (int i = 0; i < 4; ++i) {
      const uint32_t word = wg[i];
      for (int n = 0; n < 8; ++n) {
        const float v = xg[8 * i + n];
        qsum += v * (float)((word >> (4 * n)) & 15u);
        xsum += v;
      }
    }
    acc += bf16_to_f32(s[g]) * qsum;
    acc += bf16_to_f32(b[g]) * xsum;
  }
  return acc;
}

/* y[o] = bf16(row o), parallel over rows */
static void q4_project(const float* x, CmoeQ4 p, int in, int out, float* y) {
  const int words = in / 8, meta = in / 32;
#pragma omp parallel for schedule(static)
  for (int o = 0; o < out; ++o) y[o] = r16(q4_row(x, p.w + (size_t)o * words, p.s + (size_t)o * meta,
                                                   p.b + (size_t)o * meta, in));
}

static CmoeQ4 record_part(const CmoeLayer* L, int record, int proj) {
  const uint8_t* rec = L->records + (uint64_t)record * L->record_stride;
  CmoeQ4 q;
  q.w = (const uint32_t*)(rec + L->offsets[3 * proj + 0]);
  q.s = (const uint16_t*)(rec + L->offsets[3 * proj + 1]);
  q.b = (const uint16_t*)(rec + L->offsets[3 * proj + 2]);
  return q;
}

/* One decode token-layer.  x: [H] bf16 bits.  Outputs: inds [k], scores [k]
 * (bf16 values as float), y [H] bf16 bits.  scratch: at least
 * cmoe_scratch_floats() floats.  Returns 0. */
int cmoe_scratch_floats(int hidden, int inter, int experts, int top_k) {
  return hidden + 2 * experts + 4 * inter + (top_k + 2) * hidden + 64;
}

int cmoe_decode_token(const CmoeLayer* L, const uint16_t* x_bits, int32_t* inds, float* scores,
                      uint16_t* y_bits, float* scratch) {
  const int H = L->hidden, I = L->inter, E = L->experts, K = L->top_k;
  float* x = scratch;
  float* logits = x + H;
  float* gates = logits + E;
  float* g = gates + E;
  float* u = g + I;
  float* act = u + I;
  float* tmp = act + I;
  float* down = tmp + I;             /* [K, H] */
  float* shared = down + (size_t)K * H; /* [H] */
  float* yacc = shared + H;          /* [H] */
  for (int h = 0; h < H; ++h) x[h] = bf16_to_f32(x_bits[h]);

  /* router */
#pragma omp parallel for schedule(static)
  for (int e = 0; e < E; ++e) {
    const uint16_t* w = L->router + (size_t)e * H;
    float acc = 0.0f;
    for (int h = 0; h < H; ++h) acc += x[h] * bf16_to_f32(w[h]);
    if (L->router_bias) acc += L->router_bias[e];
    logits[e] = r16(acc);
  }
  float m = -INFINITY;
  for (int e = 0; e < E; ++e) m = logits[e] > m ? logits[e] : m;
  double total = 0.0;
  for (int e = 0; e < E; ++e) total += exp((double)logits[e] - (double)m);
  for (int e = 0; e < E; ++e) gates[e] = r16((float)(exp((double)logits[e] - (double)m) / total));
  /* top-k: gate descending, index ascending */
  for (int k = 0; k < K; ++k) {
    int best = -1;
    for (int e = 0; e < E; ++e) {
      int taken = 0;
      for (int j = 0; j < k; ++j) taken |= inds[j] == e;
      if (taken) continue;
      if (best < 0 || gates[e] > gates[best]) best = e;
    }
    inds[k] = best;
  }
  float mass = 0.0f;
  for (int k = 0; k < K; ++k) mass += gates[inds[k]];
  mass = r16(mass);
  for (int k = 0; k < K; ++k) scores[k] = r16(gates[inds[k]] / mass);

  /* shared expert and its gate */
  float shared_sig = 0.0f;
  if (L->shared_inter > 0) {
    const int Is = L->shared_inter;
    q4_project(x, L->sgate, H, Is, g);
    q4_project(x, L->sup, H, Is, u);
    for (int i = 0; i < Is; ++i) act[i] = swiglu_bf16(g[i], u[i]);
    q4_project(act, L->sdown, Is, H, shared);
    shared_sig = sigmoid_bf16(r16(q4_row(x, L->segate.w, L->segate.s, L->segate.b, H)));
  }
  /* routed experts */
  for (int k = 0; k < K; ++k) {
    const int rec = L->record_of ? L->record_of[inds[k]] : inds[k];
    q4_project(x, record_part(L, rec, 0), H, I, g);
    q4_project(x, record_part(L, rec, 1), H, I, u);
    for (int i = 0; i < I; ++i) act[i] = swiglu_bf16(g[i], u[i]);
    q4_project(act, record_part(L, rec, 2), I, H, down + (size_t)k * H);
  }
  (void)tmp;
  /* fused combine */
  for (int h = 0; h < H; ++h) {
    float c = 0.0f;
    for (int k = 0; k < K; ++k) {
      volatile float p = down[(size_t)k * H + h] * scores[k];
      c = c + p;
    }
    float y = r16(c);
    if (L->shared_inter > 0) y = r16(y + r16(shared_sig * shared[h]));
    yacc[h] = y;
    y_bits[h] = f32_to_bf16(y);
  }
  return 0;
}

int cmoe_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
