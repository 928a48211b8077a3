/*
 * sanitize_check.c - drives every function of the CPU oracle once on small,
 * ragged inputs (odd widths, K tails, contexts that end mid-chunk, a tiny
 * two-layer model through several decode steps), so that a build of
 * hq_oracle.c with AddressSanitizer and UndefinedBehaviorSanitizer
 * (`make -C oracle sanitize`) reports any out-of-bounds access, leak or
 * undefined operation.  TEST INFRASTRUCTURE ONLY (run by
 * tests/test_oracle_sanitize.py); it checks memory safety, not values:
 * the values are pinned by the other oracle tests.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "hq_oracle.h"

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static uint32_t next_u32(void)
{
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (uint32_t)(rng_state >> 16);
}
static float uniform(float lo, float hi) { return lo + (hi - lo) * (float)(next_u32() & 0xffffff) / 16777216.0f; }

/* exactly-sized heap buffers, so ASan sees any access one element past */
static void* xmalloc(size_t n)
{
    void* p = malloc(n ? n : 1);
    if (!p) { fprintf(stderr, "out of memory\n"); exit(2); }
    return p;
}

static uint8_t* random_packed(int rows, int width)
{
    int8_t* w = xmalloc((size_t)rows * width);
    for (size_t i = 0; i < (size_t)rows * width; ++i) w[i] = (int8_t)((int)(next_u32() % 15) - 7);
    uint8_t* p = xmalloc((size_t)rows * (width / 2));
    if (or_pack_int4(w, rows, width, p) != 0) { fprintf(stderr, "pack failed\n"); exit(1); }
    int8_t* back = xmalloc((size_t)rows * width);
    or_unpack_int4(p, rows, width, back);
    if (memcmp(back, w, (size_t)rows * width) != 0) { fprintf(stderr, "unpack mismatch\n"); exit(1); }
    free(back);
    free(w);
    return p;
}

static float* random_f32(size_t n, float lo, float hi)
{
    float* x = xmalloc(n * sizeof(float));
    for (size_t i = 0; i < n; ++i) x[i] = uniform(lo, hi);
    return x;
}

static void kernels(void)
{
    static const int widths[] = {2, 30, 62, 64, 66, 130, 2562};
    for (size_t wi = 0; wi < sizeof(widths) / sizeof(widths[0]); ++wi) {
        const int rows = 3 + (int)wi * 5, width = widths[wi];
        uint8_t* w = random_packed(rows, width);
        float* s = random_f32(rows, 0.005f, 0.02f);
        float* x = random_f32(width, -3.0f, 3.0f);
        int8_t* q = xmalloc(width);
        float* out = xmalloc(rows * sizeof(float));
        int32_t* acc = xmalloc(rows * sizeof(int32_t));
        float act = or_quantize_activation(x, width, q);
        or_int4_i8_gemv(q, w, s, act, out, rows, width);
        or_int4_i8_gemv_acc(q, w, rows, width, acc);
        or_quant_int4_gemv(x, w, s, out, rows, width, q, acc);
        const int m = 3;
        int8_t* qm = xmalloc((size_t)m * width);
        int32_t* accm = xmalloc((size_t)m * rows * sizeof(int32_t));
        for (int i = 0; i < m; ++i) memcpy(qm + (size_t)i * width, q, width);
        or_int4_i8_gemm_acc(qm, w, m, rows, width, accm);
        float* g = random_f32(width, 0.5f, 1.5f);
        float* y = xmalloc(width * sizeof(float));
        or_rmsnorm(x, g, y, width, 1e-6f);
        free(g); free(y); free(qm); free(accm);
        free(w); free(s); free(x); free(q); free(out); free(acc);
    }
    /* zero vector: the eps guard */
    float z[5] = {0};
    int8_t zq[5];
    (void)or_quantize_activation(z, 5, zq);

    /* attention at contexts ending inside and on chunk borders */
    static const int ctxs[] = {1, 7, 63, 64, 65, 200};
    for (size_t ci = 0; ci < sizeof(ctxs) / sizeof(ctxs[0]); ++ci) {
        const int ctx = ctxs[ci], kv = 2, groups = 3, d = 16;
        float* qv = random_f32((size_t)kv * groups * d, -1, 1);
        float* kf = random_f32((size_t)ctx * kv * d, -1, 1);
        float* vf = random_f32((size_t)ctx * kv * d, -1, 1);
        uint16_t* kh = xmalloc((size_t)ctx * kv * d * 2);
        uint16_t* vh = xmalloc((size_t)ctx * kv * d * 2);
        or_f32_to_f16_array(kf, kh, (int64_t)ctx * kv * d);
        or_f32_to_f16_array(vf, vh, (int64_t)ctx * kv * d);
        float* back = xmalloc((size_t)ctx * kv * d * sizeof(float));
        or_f16_to_f32_array(kh, back, (int64_t)ctx * kv * d);
        float* scores = xmalloc((size_t)kv * groups * ctx * sizeof(float));
        float* o = xmalloc((size_t)kv * groups * d * sizeof(float));
        or_gqa_decode_ref(qv, kf, vf, scores, o, ctx, kv, groups, d, ctx);
        or_gqa_decode_split(qv, kh, vh, o, ctx, kv, groups, d, (int64_t)kv * d, 64);
        or_gqa_decode_split_f32(qv, kf, vf, o, ctx, kv, groups, d, (int64_t)kv * d, 16);
        float* heads = random_f32((size_t)kv * d, -2, 2);
        float* hg = random_f32(d, 0.5f, 1.5f);
        float* cs = random_f32(d / 2, -1, 1);
        float* sn = random_f32(d / 2, -1, 1);
        or_head_norm(heads, hg, kv, d, 1e-6f);
        or_rope(heads, kv, d, cs, sn);
        free(heads); free(hg); free(cs); free(sn);
        free(qv); free(kf); free(vf); free(kh); free(vh); free(back); free(scores); free(o);
    }

    /* SwiGLU, argmax, pairwise sum, the sampler over ragged sizes */
    static const int ns[] = {1, 5, 127, 129, 4097, 9000};
    for (size_t ni = 0; ni < sizeof(ns) / sizeof(ns[0]); ++ni) {
        const int n = ns[ni];
        float* a = random_f32(n, -8, 8);
        float* b = random_f32(n, -8, 8);
        float* c = xmalloc(n * sizeof(float));
        or_swiglu(a, b, c, n);
        (void)or_argmax(c, n);
        (void)or_pairwise_sum_f32(a, n);
        const int ngen = 4;
        int32_t gen[4] = {0, n - 1, n / 2, 0};
        const int k = n < 40 ? n : 40;
        int32_t* ids = xmalloc(k * sizeof(int32_t));
        float* probs = xmalloc(k * sizeof(float));
        (void)or_sample_token(a, n, gen, ngen, 1.08f, 0.7f, 40, 0.9f, 0.37, ids, probs);
        (void)or_sample_token(a, n, gen, ngen, 1.0f, 1.0f, 1, 1e-6f, 0.99, ids, probs);
        free(ids); free(probs); free(a); free(b); free(c);
    }
}

static void model_steps(void)
{
    const int L = 2, H = 64, I = 96, heads = 4, kvh = 2, d = 16, V = 50, P = 16;
    const int qkv = heads * d + 2 * kvh * d;
    or_layer* layers = xmalloc(sizeof(or_layer) * L);
    void* owned[64];
    int no = 0;
#define OWN(p) (owned[no++] = (void*)(p))
    for (int l = 0; l < L; ++l) {
        or_layer* ly = &layers[l];
        ly->qkv = OWN(random_packed(qkv, H));
        ly->qkv_scales = OWN(random_f32(qkv, 0.005f, 0.02f));
        ly->o = OWN(random_packed(H, heads * d));
        ly->o_scales = OWN(random_f32(H, 0.005f, 0.02f));
        ly->gate_up = OWN(random_packed(2 * I, H));
        ly->gate_up_scales = OWN(random_f32(2 * I, 0.005f, 0.02f));
        ly->down = OWN(random_packed(H, I));
        ly->down_scales = OWN(random_f32(H, 0.005f, 0.02f));
        ly->input_norm = OWN(random_f32(H, 0.5f, 1.5f));
        ly->post_norm = OWN(random_f32(H, 0.5f, 1.5f));
        ly->q_norm = OWN(random_f32(d, 0.5f, 1.5f));
        ly->k_norm = OWN(random_f32(d, 0.5f, 1.5f));
    }
    or_model m;
    memset(&m, 0, sizeof(m));
    m.layers = L; m.hidden = H; m.intermediate = I; m.heads = heads; m.kv_heads = kvh;
    m.head_dim = d; m.vocab = V; m.rope_positions = P; m.eps = 1e-6f; m.chunk = 4;
    m.layer = layers;
    m.embedding = OWN(random_packed(V, H));
    m.embedding_scales = OWN(random_f32(V, 0.005f, 0.02f));
    m.final_norm = OWN(random_f32(H, 0.5f, 1.5f));
    m.rope_cos = OWN(random_f32((size_t)P * d / 2, -1, 1));
    m.rope_sin = OWN(random_f32((size_t)P * d / 2, -1, 1));
    for (int kv_f32 = 0; kv_f32 < 2; ++kv_f32) {
        const int cap = 9;
        const size_t kv_elems = (size_t)L * cap * kvh * d;
        or_state s;
        memset(&s, 0, sizeof(s));
        s.capacity = cap;
        s.kv_f32 = kv_f32;
        s.keys = xmalloc(kv_elems * (kv_f32 ? 4 : 2));
        s.values = xmalloc(kv_elems * (kv_f32 ? 4 : 2));
        s.x = xmalloc(H * sizeof(float));
        s.logits = xmalloc(V * sizeof(float));
        s.trace = xmalloc((size_t)L * H * sizeof(float));
        int token = 3;
        for (int step = 0; step < cap; ++step) {
            token = or_forward_token(&m, &s, token);
            if (token < 0) { fprintf(stderr, "step %d failed\n", step); exit(1); }
        }
        /* a full cache and an out-of-vocabulary token are refused, not run */
        if (or_forward_token(&m, &s, token) != -1) { fprintf(stderr, "full cache not refused\n"); exit(1); }
        s.position = 0;
        if (or_forward_token(&m, &s, V) != -2) { fprintf(stderr, "bad token not refused\n"); exit(1); }
        float* e = xmalloc(H * sizeof(float));
        or_embedding(&m, V - 1, e);
        free(e);
        free(s.keys); free(s.values); free(s.x); free(s.logits); free(s.trace);
    }
    for (int i = 0; i < no; ++i) free(owned[i]);
    free(layers);
#undef OWN
}

int main(void)
{
    (void)or_expf(-100.0f);
    (void)or_expf(88.0f);
    (void)or_f32_to_f16(65520.0f);
    (void)or_f16_to_f32(0x7c01);
    kernels();
    model_steps();
    printf("sanitize_check: ok\n");
    return 0;
}
