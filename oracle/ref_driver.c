/*
 * ref_driver.c -- test-only harness compiled together with the reference's own
 * sources (src/quant.c, src/kernels.c, src/runtime.c, src/model.c, src/gguf.c,
 * src/threadpool.c, built where they lie) into oracle/_ref/libqref_*.so.
 *
 * TEST INFRASTRUCTURE ONLY.  It exposes the reference's static-inline fp16
 * helpers and KernelOps function pointers as plain exported symbols, and runs
 * the reference's MoE block (which only exists inline in forward_runtime,
 * src/runtime.c:202-269) on caller-supplied tensors through a one-layer
 * in-memory Transformer.  Nothing here computes; every number comes from the
 * reference's own code.
 */
#define _POSIX_C_SOURCE 199309L
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "kernels.h"
#include "model.h"
#include "quant.h"
#include "runtime.h"
#include "types.h"

float refdrv_h2f(uint16_t h) { return fp16_to_fp32(h); }
/* Batch form: writes through memory so NaN payloads keep their bits. */
void refdrv_h2f_batch(const uint16_t* h, float* out, long n) {
    long i;
    for (i = 0; i < n; i++) out[i] = fp16_to_fp32(h[i]);
}
uint16_t refdrv_f2h(float f) { return fp32_to_fp16(f); }

int refdrv_has_avx2_paths(void) {
#if defined(__AVX2__)
    return 1;
#else
    return 0;
#endif
}

int refdrv_has_avx512_paths(void) {
#if defined(__AVX512F__)
    return 1;
#else
    return 0;
#endif
}

/* matmul_q_fused called from this file: in the GPU-bound builds
 * (ref_gpu_bind.c) the linker sends it to qr_matmul_q_fused, in the plain
 * builds it is the reference's own. */
void refdrv_matmul_q_fused(float* out, const float* x, const void* w, uint32_t type, int n, int d,
                           int threads) {
    matmul_q_fused(out, x, w, type, n, d, threads);
}

/* KernelOps.matmul / softmax / rmsnorm of a backend (src/kernels.c:209-214). */
void refdrv_matmul(int backend, float* out, const float* x, const float* w, int n, int d) {
    kernels_for_backend((KernelBackend)backend)->matmul(out, x, w, n, d, 1);
}
void refdrv_softmax(int backend, float* x, int n) {
    kernels_for_backend((KernelBackend)backend)->softmax(x, n);
}
void refdrv_rmsnorm(int backend, float* o, const float* x, const float* w, int n) {
    kernels_for_backend((KernelBackend)backend)->rmsnorm(o, x, w, n);
}

/*
 * Run the reference's forward_runtime on a one-layer MoE model for T tokens.
 * Token t's embedding row is x_in[t] (an F32 table); attention weights are
 * NULL so the attention block adds exactly zero; the MoE input is therefore
 * xb = rmsnorm(x_in[t]) with unit weights, returned in xb_out[t], and the
 * residual after the MoE block is returned in x_out[t].  The backend picks the
 * router's KernelOps.matmul order; threads is the OpenMP width of
 * matmul_q_fused.  Experts are [E][rows][cols] tensors sliced as
 * src/model.c:412-419 does.
 */
int refdrv_moe_layer(const float* x_in, float* xb_out, float* x_out, int T, int dim, int hidden,
                     int E, int K, const float* router, const void* up, uint32_t up_type,
                     const void* gate, uint32_t gate_type, const void* down, uint32_t down_type,
                     int backend, int threads) {
    Transformer t;
    RuntimeContext rt;
    RuntimeOptions opt;
    float* ones;
    float* rms_att[1];
    float* rms_ffn[1];
    float* null_l[1] = {NULL};
    float* router_l[1];
    float** ew1[1];
    float** ew2[1];
    float** ew3[1];
    uint32_t t_up[1], t_down[1], t_gate[1];
    size_t s_up, s_down, s_gate;
    int e, tok;

    if (E > 256 || K > 16 || K > E) return -1;
    memset(&t, 0, sizeof(t));
    t.config.dim = dim;
    t.config.hidden_dim = hidden;
    t.config.n_layers = 1;
    /* forward_runtime's attention holds one head's key row in a 512-float
     * stack buffer (src/runtime.c:145): keep head_dim = dim / n_heads <= 512.
     * With NULL attention weights the heads add exactly zero either way. */
    t.config.n_heads = 1;
    while (dim / t.config.n_heads > 512 || dim % t.config.n_heads) t.config.n_heads++;
    t.config.n_kv_heads = t.config.n_heads;
    t.config.vocab_size = 1;
    t.config.seq_len = 1;
    t.config.rope_freq_base = 10000.0f;
    t.config.expert_count = E;
    t.config.expert_used_count = K;

    ones = (float*)malloc((size_t)dim * sizeof(float));
    ew1[0] = (float**)malloc((size_t)E * sizeof(float*));
    ew2[0] = (float**)malloc((size_t)E * sizeof(float*));
    ew3[0] = (float**)malloc((size_t)E * sizeof(float*));
    if (!ones || !ew1[0] || !ew2[0] || !ew3[0]) return -2;
    for (e = 0; e < dim; e++) ones[e] = 1.0f;

    s_up = (up_type == 8 ? (size_t)(dim / 32) * 34 : up_type == 12 ? (size_t)(dim / 256) * 144
            : up_type == 13 ? (size_t)(dim / 256) * 176 : up_type == 14 ? (size_t)(dim / 256) * 210
            : (size_t)dim * 4) * (size_t)hidden;
    s_gate = (gate_type == 8 ? (size_t)(dim / 32) * 34 : gate_type == 12 ? (size_t)(dim / 256) * 144
              : gate_type == 13 ? (size_t)(dim / 256) * 176 : gate_type == 14 ? (size_t)(dim / 256) * 210
              : (size_t)dim * 4) * (size_t)hidden;
    s_down = (down_type == 8 ? (size_t)(hidden / 32) * 34 : down_type == 12 ? (size_t)(hidden / 256) * 144
              : down_type == 13 ? (size_t)(hidden / 256) * 176 : down_type == 14 ? (size_t)(hidden / 256) * 210
              : (size_t)hidden * 4) * (size_t)dim;
    for (e = 0; e < E; e++) {
        ew1[0][e] = (float*)((const char*)up + (size_t)e * s_up);
        ew3[0][e] = (float*)((const char*)gate + (size_t)e * s_gate);
        ew2[0][e] = (float*)((const char*)down + (size_t)e * s_down);
    }
    rms_att[0] = ones;
    rms_ffn[0] = ones;
    router_l[0] = (float*)router;
    t_up[0] = up_type;
    t_down[0] = down_type;
    t_gate[0] = gate_type;

    t.weights.token_embedding_table = (float*)x_in;
    t.weights.token_embd_type = 0;
    t.weights.token_embd_row_bytes = (size_t)dim * sizeof(float);
    t.weights.rms_att_weight = rms_att;
    t.weights.rms_ffn_weight = rms_ffn;
    t.weights.wq = null_l;
    t.weights.wk = null_l;
    t.weights.wv = null_l;
    t.weights.wo = null_l;
    t.weights.rms_final_weight = ones;
    t.weights.wcls = NULL;
    t.weights.ffn_gate_inp = router_l;
    t.weights.expert_w1 = ew1;
    t.weights.expert_w2 = ew2;
    t.weights.expert_w3 = ew3;
    t.weights.exp_w1_type = t_up;
    t.weights.exp_w2_type = t_down;
    t.weights.exp_w3_type = t_gate;
    malloc_run_state(&t.state, &t.config);

    memset(&opt, 0, sizeof(opt));
    opt.backend = (KernelBackend)backend;
    opt.num_threads = threads;
    runtime_init(&rt, opt);

    for (tok = 0; tok < T; tok++) {
        if (xb_out) {
            rt.kernels->rmsnorm(xb_out + (size_t)tok * dim, x_in + (size_t)tok * dim, ones, dim);
        }
        forward_runtime(&rt, &t, tok, 0);
        if (x_out) memcpy(x_out + (size_t)tok * dim, t.state.x, (size_t)dim * sizeof(float));
    }

    free_run_state(&t.state);
    free(ones);
    free(ew1[0]);
    free(ew2[0]);
    free(ew3[0]);
    return 0;
}

/*
 * Timing of the reference's MoE block for the CPU baseline: a one-layer model
 * whose layer weights rotate over `nlayers` copies (copy l: router_l[l],
 * up_l[l], gate_l[l], down_l[l], each an [E][rows][cols] tensor), built once
 * outside the timed region (malloc_run_state and runtime_init included), then
 * `warmup` untimed and `reps` timed forward_runtime calls; call i runs copy
 * i % nlayers on token row x_in[i % T].  times[r] receives call r's
 * CLOCK_MONOTONIC seconds.  One layer per call, fed from the embedding row:
 * the reference's Q4_K dot returns invalid values, which a second layer's
 * router would turn into an out-of-range expert index.
 */
int refdrv_moe_bench(const float* x_in, int T, int dim, int hidden, int E, int K, int nlayers,
                     const float* const* router_l, const void* const* up_l, uint32_t up_type,
                     const void* const* gate_l, uint32_t gate_type, const void* const* down_l,
                     uint32_t down_type, int backend, int threads, int warmup, int reps,
                     double* times) {
    Transformer t;
    RuntimeContext rt;
    RuntimeOptions opt;
    float *ones, **rms, **nulls, **router;
    float ***ew1, ***ew2, ***ew3;
    uint32_t *t_up, *t_down, *t_gate;
    size_t s_up, s_gate, s_down;
    int l, e, i;
    struct timespec a, b;

    if (E > 256 || K > 16 || K > E || nlayers < 1 || T < 1) return -1;
    memset(&t, 0, sizeof(t));
    t.config.dim = dim;
    t.config.hidden_dim = hidden;
    t.config.n_layers = 1;
    t.config.n_heads = 1;
    while (dim / t.config.n_heads > 512 || dim % t.config.n_heads) t.config.n_heads++;
    t.config.n_kv_heads = t.config.n_heads;
    t.config.vocab_size = 1;
    t.config.seq_len = 1;
    t.config.rope_freq_base = 10000.0f;
    t.config.expert_count = E;
    t.config.expert_used_count = K;

    ones = (float*)malloc((size_t)dim * sizeof(float));
    rms = (float**)malloc((size_t)nlayers * sizeof(float*));
    nulls = (float**)calloc((size_t)nlayers, sizeof(float*));
    router = (float**)malloc((size_t)nlayers * sizeof(float*));
    ew1 = (float***)malloc((size_t)nlayers * sizeof(float**));
    ew2 = (float***)malloc((size_t)nlayers * sizeof(float**));
    ew3 = (float***)malloc((size_t)nlayers * sizeof(float**));
    t_up = (uint32_t*)malloc((size_t)nlayers * sizeof(uint32_t));
    t_down = (uint32_t*)malloc((size_t)nlayers * sizeof(uint32_t));
    t_gate = (uint32_t*)malloc((size_t)nlayers * sizeof(uint32_t));
    if (!ones || !rms || !nulls || !router || !ew1 || !ew2 || !ew3 || !t_up || !t_down || !t_gate)
        return -2;
    for (i = 0; i < dim; i++) ones[i] = 1.0f;
    s_up = (up_type == 8 ? (size_t)(dim / 32) * 34 : up_type == 12 ? (size_t)(dim / 256) * 144
            : up_type == 13 ? (size_t)(dim / 256) * 176 : (size_t)(dim / 256) * 210) * (size_t)hidden;
    s_gate = (gate_type == 8 ? (size_t)(dim / 32) * 34 : gate_type == 12 ? (size_t)(dim / 256) * 144
              : gate_type == 13 ? (size_t)(dim / 256) * 176 : (size_t)(dim / 256) * 210) * (size_t)hidden;
    s_down = (down_type == 8 ? (size_t)(hidden / 32) * 34 : down_type == 12 ? (size_t)(hidden / 256) * 144
              : down_type == 13 ? (size_t)(hidden / 256) * 176 : (size_t)(hidden / 256) * 210) * (size_t)dim;
    for (l = 0; l < nlayers; l++) {
        rms[l] = ones;
        router[l] = (float*)router_l[l];
        ew1[l] = (float**)malloc((size_t)E * sizeof(float*));
        ew2[l] = (float**)malloc((size_t)E * sizeof(float*));
        ew3[l] = (float**)malloc((size_t)E * sizeof(float*));
        if (!ew1[l] || !ew2[l] || !ew3[l]) return -2;
        for (e = 0; e < E; e++) {
            ew1[l][e] = (float*)((const char*)up_l[l] + (size_t)e * s_up);
            ew3[l][e] = (float*)((const char*)gate_l[l] + (size_t)e * s_gate);
            ew2[l][e] = (float*)((const char*)down_l[l] + (size_t)e * s_down);
        }
        t_up[l] = up_type;
        t_down[l] = down_type;
        t_gate[l] = gate_type;
    }
    t.weights.token_embedding_table = (float*)x_in;
    t.weights.token_embd_type = 0;
    t.weights.token_embd_row_bytes = (size_t)dim * sizeof(float);
    t.weights.rms_att_weight = rms;
    t.weights.rms_ffn_weight = rms;
    t.weights.wq = nulls;
    t.weights.wk = nulls;
    t.weights.wv = nulls;
    t.weights.wo = nulls;
    t.weights.rms_final_weight = ones;
    t.weights.wcls = NULL;
    t.weights.ffn_gate_inp = router;
    t.weights.expert_w1 = ew1;
    t.weights.expert_w2 = ew2;
    t.weights.expert_w3 = ew3;
    t.weights.exp_w1_type = t_up;
    t.weights.exp_w2_type = t_down;
    t.weights.exp_w3_type = t_gate;
    malloc_run_state(&t.state, &t.config);
    memset(&opt, 0, sizeof(opt));
    opt.backend = (KernelBackend)backend;
    opt.num_threads = threads;
    runtime_init(&rt, opt);

    for (i = 0; i < warmup + reps; i++) {
        l = i % nlayers;  /* the layer's weights: copy l */
        t.weights.ffn_gate_inp = router + l;
        t.weights.expert_w1 = ew1 + l;
        t.weights.expert_w2 = ew2 + l;
        t.weights.expert_w3 = ew3 + l;
        t.weights.exp_w1_type = t_up + l;
        t.weights.exp_w2_type = t_down + l;
        t.weights.exp_w3_type = t_gate + l;
        clock_gettime(CLOCK_MONOTONIC, &a);
        forward_runtime(&rt, &t, i % T, 0);
        clock_gettime(CLOCK_MONOTONIC, &b);
        if (i >= warmup)
            times[i - warmup] = (double)(b.tv_sec - a.tv_sec) + 1e-9 * (double)(b.tv_nsec - a.tv_nsec);
    }

    free_run_state(&t.state);
    for (l = 0; l < nlayers; l++) {
        free(ew1[l]);
        free(ew2[l]);
        free(ew3[l]);
    }
    free(ones);
    free(rms);
    free(nulls);
    free(router);
    free(ew1);
    free(ew2);
    free(ew3);
    free(t_up);
    free(t_down);
    free(t_gate);
    return 0;
}

/*
 * Timing of one decoder layer of forward_runtime at position `pos`, for the
 * CPU baseline of the decode step: a one-layer model (RMSNorm, Q/K/V, RoPE,
 * the attention over pos + 1 cached positions, Wo, RMSNorm, the MoE block)
 * whose weights rotate over `ncopies` copies (copy c: wq[c] .. wo[c] of types
 * wtype[0..3], router[c], up[c] / gate[c] / down[c] as [E][rows][cols]); the
 * fp32 KV cache rows 0 .. pos-1 hold seeded values in [-0.5, 0.5); wcls is
 * NULL, so the lm_head costs nothing here (the caller times it alone).
 * head_dim is dim / n_heads, as the reference fixes it.  Call i embeds token
 * i % n_tok of tok_embd (fp32 rows) at position pos.  times[r] receives
 * call r's CLOCK_MONOTONIC seconds after `warmup` untimed calls.
 */
int refdrv_decode_layer_bench(int dim, int n_heads, int n_kv_heads, int hidden, int E, int K,
                              int pos, int ncopies, const float* tok_embd, int n_tok,
                              const void* const* wq, const void* const* wk,
                              const void* const* wv, const void* const* wo,
                              const uint32_t* wtype, const float* const* router,
                              const void* const* up, uint32_t up_type, const void* const* gate,
                              const void* const* down, uint32_t down_type, const float* rms,
                              int backend, int threads, int warmup, int reps, double* times) {
    Transformer t;
    RuntimeContext rt;
    RuntimeOptions opt;
    float **rmsp, **qp, **kp, **vp, **op, **rp;
    float ***ew1, ***ew2, ***ew3;
    uint32_t *tq, *tk, *tv, *to, *t_up, *t_down, *t_gate;
    size_t s_up, s_down, kv_dim, i, r;
    int l, e, c;
    struct timespec a, b;
    uint64_t h = 0x9E3779B97F4A7C15ull;

    if (E < 1 || E > 256 || K > 16 || K > E || ncopies < 1 || n_tok < 1 || pos < 0) return -1;
    memset(&t, 0, sizeof(t));
    t.config.dim = dim;
    t.config.hidden_dim = hidden;
    t.config.n_layers = 1;
    t.config.n_heads = n_heads;
    t.config.n_kv_heads = n_kv_heads;
    t.config.vocab_size = 1;
    t.config.seq_len = pos + 1;
    t.config.rope_freq_base = 1000000.0f;
    t.config.expert_count = E;
    t.config.expert_used_count = K;
    rmsp = (float**)malloc((size_t)ncopies * 6 * sizeof(float*));
    ew1 = (float***)malloc((size_t)ncopies * 3 * sizeof(float**));
    tq = (uint32_t*)malloc((size_t)ncopies * 7 * sizeof(uint32_t));
    if (!rmsp || !ew1 || !tq) return -2;
    qp = rmsp + ncopies;
    kp = qp + ncopies;
    vp = kp + ncopies;
    op = vp + ncopies;
    rp = op + ncopies;
    ew2 = ew1 + ncopies;
    ew3 = ew2 + ncopies;
    tk = tq + ncopies;
    tv = tk + ncopies;
    to = tv + ncopies;
    t_up = to + ncopies;
    t_down = t_up + ncopies;
    t_gate = t_down + ncopies;
    s_up = (up_type == 8 ? (size_t)(dim / 32) * 34 : up_type == 12 ? (size_t)(dim / 256) * 144
            : up_type == 13 ? (size_t)(dim / 256) * 176 : (size_t)(dim / 256) * 210) * (size_t)hidden;
    s_down = (down_type == 8 ? (size_t)(hidden / 32) * 34 : down_type == 12 ? (size_t)(hidden / 256) * 144
              : down_type == 13 ? (size_t)(hidden / 256) * 176 : (size_t)(hidden / 256) * 210) * (size_t)dim;
    for (c = 0; c < ncopies; c++) {
        rmsp[c] = (float*)rms;
        qp[c] = (float*)wq[c];
        kp[c] = (float*)wk[c];
        vp[c] = (float*)wv[c];
        op[c] = (float*)wo[c];
        rp[c] = (float*)router[c];
        tq[c] = wtype[0];
        tk[c] = wtype[1];
        tv[c] = wtype[2];
        to[c] = wtype[3];
        t_up[c] = t_gate[c] = up_type;
        t_down[c] = down_type;
        ew1[c] = (float**)malloc((size_t)E * 3 * sizeof(float*));
        if (!ew1[c]) return -2;
        ew2[c] = ew1[c] + E;
        ew3[c] = ew2[c] + E;
        for (e = 0; e < E; e++) {
            ew1[c][e] = (float*)((const char*)up[c] + (size_t)e * s_up);
            ew3[c][e] = (float*)((const char*)gate[c] + (size_t)e * s_up);
            ew2[c][e] = (float*)((const char*)down[c] + (size_t)e * s_down);
        }
    }
    t.weights.token_embedding_table = (float*)tok_embd;
    t.weights.token_embd_type = 0;
    t.weights.token_embd_row_bytes = (size_t)dim * sizeof(float);
    t.weights.rms_final_weight = (float*)rms;
    t.weights.wcls = NULL;
    malloc_run_state(&t.state, &t.config);
    /* the cache rows before pos (row t at t * dim floats; kv_dim of them read) */
    kv_dim = (size_t)n_kv_heads * (size_t)(dim / n_heads);
    for (r = 0; r < (size_t)pos; r++)
        for (i = 0; i < kv_dim; i++) {
            h = h * 6364136223846793005ull + 1442695040888963407ull;
            ((float*)t.state.key_cache)[r * (size_t)dim + i] = (float)(h >> 40) * 0x1p-24f - 0.5f;
            h = h * 6364136223846793005ull + 1442695040888963407ull;
            ((float*)t.state.value_cache)[r * (size_t)dim + i] = (float)(h >> 40) * 0x1p-24f - 0.5f;
        }
    memset(&opt, 0, sizeof(opt));
    opt.backend = (KernelBackend)backend;
    opt.num_threads = threads;
    runtime_init(&rt, opt);
    for (i = 0; i < (size_t)(warmup + reps); i++) {
        c = (int)(i % (size_t)ncopies);
        t.weights.rms_att_weight = rmsp + c;
        t.weights.rms_ffn_weight = rmsp + c;
        t.weights.wq = qp + c;
        t.weights.wk = kp + c;
        t.weights.wv = vp + c;
        t.weights.wo = op + c;
        t.weights.wq_type = tq + c;
        t.weights.wk_type = tk + c;
        t.weights.wv_type = tv + c;
        t.weights.wo_type = to + c;
        t.weights.ffn_gate_inp = rp + c;
        t.weights.expert_w1 = ew1 + c;
        t.weights.expert_w2 = ew2 + c;
        t.weights.expert_w3 = ew3 + c;
        t.weights.exp_w1_type = t_up + c;
        t.weights.exp_w2_type = t_down + c;
        t.weights.exp_w3_type = t_gate + c;
        clock_gettime(CLOCK_MONOTONIC, &a);
        forward_runtime(&rt, &t, (int)(i % (size_t)n_tok), pos);
        clock_gettime(CLOCK_MONOTONIC, &b);
        if ((int)i >= warmup)
            times[i - (size_t)warmup] =
                (double)(b.tv_sec - a.tv_sec) + 1e-9 * (double)(b.tv_nsec - a.tv_nsec);
    }
    free_run_state(&t.state);
    for (c = 0; c < ncopies; c++) free(ew1[c]);
    free(rmsp);
    free(ew1);
    free(tq);
    (void)l;
    return 0;
}

/* CLOCK_MONOTONIC seconds of each of `reps` matmul_q_fused calls after
 * `warmup` untimed ones; call i uses weight copy i % ncopies. */
int refdrv_gemv_bench(const float* x, const void* const* w_copies, int ncopies, uint32_t type,
                      int n, int d, int threads, int warmup, int reps, float* out,
                      double* times) {
    struct timespec a, b;
    int i;
    if (ncopies < 1) return -1;
    for (i = 0; i < warmup + reps; i++) {
        clock_gettime(CLOCK_MONOTONIC, &a);
        matmul_q_fused(out, x, w_copies[i % ncopies], type, n, d, threads);
        clock_gettime(CLOCK_MONOTONIC, &b);
        if (i >= warmup)
            times[i - warmup] = (double)(b.tv_sec - a.tv_sec) + 1e-9 * (double)(b.tv_nsec - a.tv_nsec);
    }
    return 0;
}

/*
 * The reference's forward_runtime on a caller-supplied model, for n_tokens
 * tokens at positions 0 .. n_tokens-1 (the KV cache fills as it goes).
 * Per-layer tensors are arrays of L pointers (NULL allowed where the reference
 * allows it); wtype[l * 4 + {0,1,2,3}] are the types of wq, wk, wv, wo; MoE
 * experts are [E][rows][cols] tensors sliced as src/model.c:412-419 does; with
 * E = 0 up / gate / down are the dense FFN's w1 / w3 / w2 per layer.
 * kv_type: the reference's RunState.kv_cache_type (0 fp32, 1 fp16).
 * logits_out: [n_tokens][vocab]; x_out (optional): the residual after the
 * last layer, [n_tokens][dim].
 */
int refdrv_forward(int dim, int hidden, int n_layers, int n_heads, int n_kv_heads, int vocab,
                   int seq_len, float rope_base, int E, int K, const void* tok_embd,
                   uint32_t tok_type, size_t tok_row_bytes, const float* const* rms_att,
                   const float* const* rms_ffn, const void* const* wq, const void* const* wk,
                   const void* const* wv, const void* const* wo, const uint32_t* wtype,
                   const float* const* router, const void* const* up, const void* const* gate,
                   const void* const* down, uint32_t up_type, uint32_t gate_type,
                   uint32_t down_type, const float* rms_final, const void* wcls,
                   uint32_t wcls_type, const int* tokens, int n_tokens, int kv_type, int backend,
                   int threads, float* logits_out, float* x_out) {
    Transformer t;
    RuntimeContext rt;
    RuntimeOptions opt;
    float ***ew1, ***ew2, ***ew3;
    uint32_t *tq, *tk, *tv, *to, *t_up, *t_down, *t_gate;
    size_t s_up, s_gate, s_down;
    int l, e, i;

    if (E > 256 || K > 16 || K > E) return -1;
    memset(&t, 0, sizeof(t));
    t.config.dim = dim;
    t.config.hidden_dim = hidden;
    t.config.n_layers = n_layers;
    t.config.n_heads = n_heads;
    t.config.n_kv_heads = n_kv_heads;
    t.config.vocab_size = vocab;
    t.config.seq_len = seq_len;
    t.config.rope_freq_base = rope_base;
    t.config.expert_count = E;
    t.config.expert_used_count = K;

    ew1 = (float***)malloc((size_t)n_layers * sizeof(float**));
    ew2 = (float***)malloc((size_t)n_layers * sizeof(float**));
    ew3 = (float***)malloc((size_t)n_layers * sizeof(float**));
    tq = (uint32_t*)malloc((size_t)n_layers * sizeof(uint32_t) * 7);
    if (!ew1 || !ew2 || !ew3 || !tq) return -2;
    tk = tq + n_layers;
    tv = tk + n_layers;
    to = tv + n_layers;
    t_up = to + n_layers;
    t_down = t_up + n_layers;
    t_gate = t_down + n_layers;
    s_up = (up_type == 8 ? (size_t)(dim / 32) * 34 : up_type == 12 ? (size_t)(dim / 256) * 144
            : up_type == 13 ? (size_t)(dim / 256) * 176 : up_type == 14 ? (size_t)(dim / 256) * 210
            : (size_t)dim * 4) * (size_t)hidden;
    s_gate = (gate_type == 8 ? (size_t)(dim / 32) * 34 : gate_type == 12 ? (size_t)(dim / 256) * 144
              : gate_type == 13 ? (size_t)(dim / 256) * 176 : gate_type == 14 ? (size_t)(dim / 256) * 210
              : (size_t)dim * 4) * (size_t)hidden;
    s_down = (down_type == 8 ? (size_t)(hidden / 32) * 34 : down_type == 12 ? (size_t)(hidden / 256) * 144
              : down_type == 13 ? (size_t)(hidden / 256) * 176 : down_type == 14 ? (size_t)(hidden / 256) * 210
              : (size_t)hidden * 4) * (size_t)dim;
    for (l = 0; l < n_layers; l++) {
        tq[l] = wtype[4 * l];
        tk[l] = wtype[4 * l + 1];
        tv[l] = wtype[4 * l + 2];
        to[l] = wtype[4 * l + 3];
        t_up[l] = up_type;
        t_down[l] = down_type;
        t_gate[l] = gate_type;
        ew1[l] = ew2[l] = ew3[l] = NULL;
        if (E > 0) {
            ew1[l] = (float**)malloc((size_t)E * sizeof(float*));
            ew2[l] = (float**)malloc((size_t)E * sizeof(float*));
            ew3[l] = (float**)malloc((size_t)E * sizeof(float*));
            if (!ew1[l] || !ew2[l] || !ew3[l]) return -2;
            for (e = 0; e < E; e++) {
                ew1[l][e] = (float*)((const char*)up[l] + (size_t)e * s_up);
                ew3[l][e] = (float*)((const char*)gate[l] + (size_t)e * s_gate);
                ew2[l][e] = (float*)((const char*)down[l] + (size_t)e * s_down);
            }
        }
    }
    t.weights.token_embedding_table = (float*)tok_embd;
    t.weights.token_embd_type = tok_type;
    t.weights.token_embd_row_bytes = tok_row_bytes;
    t.weights.rms_att_weight = (float**)rms_att;
    t.weights.rms_ffn_weight = (float**)rms_ffn;
    t.weights.wq = (float**)wq;
    t.weights.wk = (float**)wk;
    t.weights.wv = (float**)wv;
    t.weights.wo = (float**)wo;
    t.weights.wq_type = tq;
    t.weights.wk_type = tk;
    t.weights.wv_type = tv;
    t.weights.wo_type = to;
    t.weights.rms_final_weight = (float*)rms_final;
    t.weights.wcls = (float*)wcls;
    t.weights.wcls_type = wcls_type;
    t.weights.ffn_gate_inp = (float**)router;
    t.weights.expert_w1 = ew1;
    t.weights.expert_w2 = ew2;
    t.weights.expert_w3 = ew3;
    t.weights.exp_w1_type = t_up;
    t.weights.exp_w2_type = t_down;
    t.weights.exp_w3_type = t_gate;
    if (E == 0) { /* a dense model: w1 = ffn_up, w3 = ffn_gate, w2 = ffn_down (src/model.c:434-446) */
        t.weights.w1 = (float**)up;
        t.weights.w3 = (float**)gate;
        t.weights.w2 = (float**)down;
        t.weights.w1_type = t_up;
        t.weights.w3_type = t_gate;
        t.weights.w2_type = t_down;
    }
    if (kv_type == 0) malloc_run_state(&t.state, &t.config);
    else malloc_run_state_kv(&t.state, &t.config, kv_type);
    memset(&opt, 0, sizeof(opt));
    opt.backend = (KernelBackend)backend;
    opt.num_threads = threads;
    runtime_init(&rt, opt);

    for (i = 0; i < n_tokens; i++) {
        float* lg = forward_runtime(&rt, &t, tokens[i], i);
        memcpy(logits_out + (size_t)i * vocab, lg, (size_t)vocab * sizeof(float));
        if (x_out) memcpy(x_out + (size_t)i * dim, t.state.x, (size_t)dim * sizeof(float));
    }
    free_run_state(&t.state);
    for (l = 0; l < n_layers; l++) {
        free(ew1[l]);
        free(ew2[l]);
        free(ew3[l]);
    }
    free(ew1);
    free(ew2);
    free(ew3);
    free(tq);
    return 0;
}

/* ---- GGUF (src/gguf.c, src/model.c:253-449) ------------------------------ */
#include "gguf.h"

/* gguf_init_from_buffer on the caller's bytes.  hdr receives version,
 * tensor_count, kv_count, alignment, data_offset; for the first max_t tensors:
 * the name (NUL-terminated, 96 bytes per entry, truncated), type, n_dims, ne[4]
 * and the data pointer's offset from buf.  Returns 0, or -1 when the
 * reference's parser refuses the buffer. */
int refdrv_gguf_parse(void* buf, size_t size, uint64_t* hdr, int max_t, char* names,
                      uint32_t* types, uint32_t* ndims, uint64_t* ne, uint64_t* data_off) {
    gguf_context* g = gguf_init_from_buffer(buf, size);
    uint64_t i;
    if (!g) return -1;
    hdr[0] = g->version;
    hdr[1] = g->tensor_count;
    hdr[2] = g->kv_count;
    hdr[3] = g->alignment;
    hdr[4] = g->data_offset;
    for (i = 0; i < g->tensor_count && (int)i < max_t; i++) {
        int j;
        strncpy(names + 96 * i, g->tensors[i].name, 95);
        names[96 * i + 95] = '\0';
        types[i] = g->tensors[i].type;
        ndims[i] = g->tensors[i].n_dims;
        for (j = 0; j < 4; j++) ne[4 * i + j] = g->tensors[i].ne[j];
        data_off[i] = (uint64_t)((const char*)g->tensors[i].data - (const char*)buf);
    }
    gguf_free(g);
    return 0;
}

/* gguf_get_val_u32 / _f32 / _str of one key (the string copied into out,
 * cap bytes; "" when absent).  Returns -1 when the buffer does not parse. */
int refdrv_gguf_vals(void* buf, size_t size, const char* key, uint32_t def_u32, float def_f32,
                     uint32_t* u32, float* f32, char* out, int cap) {
    gguf_context* g = gguf_init_from_buffer(buf, size);
    const char* s;
    if (!g) return -1;
    *u32 = gguf_get_val_u32(g, key, def_u32);
    *f32 = gguf_get_val_f32(g, key, def_f32);
    s = gguf_get_val_str(g, key);
    out[0] = '\0';
    if (s && cap > 0) {
        strncpy(out, s, (size_t)cap - 1);
        out[cap - 1] = '\0';
    }
    gguf_free(g);
    return 0;
}

/* load_transformer (src/model.c:451-481) of a .gguf file: cfg receives dim,
 * hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len,
 * expert_count, expert_used_count; rope the freq base.  off receives the file
 * offset of every weight pointer the loader set (-1 when NULL), in this order:
 * token_embedding_table, rms_final_weight, wcls, then per layer rms_att, rms_ffn,
 * wq, wk, wv, wo, ffn_gate_inp, then per layer and expert w1, w2, w3 (a dense
 * model: per layer its w1, w2, w3).  types: token_embd_type, wcls_type, then
 * per layer wq, wk, wv, wo, exp_w1, exp_w2, exp_w3 types (a dense model: w1,
 * w2, w3); row_bytes: token_embd_row_bytes.  The file must be a valid GGUF
 * model (the reference exits otherwise). */
int refdrv_load_gguf(const char* path, int* cfg, float* rope, int64_t* off, uint32_t* types,
                     uint64_t* row_bytes) {
    Transformer t;
    int l, e, n = 0, m = 0;
    const char* base;
    load_transformer(&t, path);
    base = (const char*)t.mapped_data;
#define OFF(p) ((p) ? (int64_t)((const char*)(p) - base) : (int64_t)-1)
    cfg[0] = t.config.dim;
    cfg[1] = t.config.hidden_dim;
    cfg[2] = t.config.n_layers;
    cfg[3] = t.config.n_heads;
    cfg[4] = t.config.n_kv_heads;
    cfg[5] = t.config.vocab_size;
    cfg[6] = t.config.seq_len;
    cfg[7] = t.config.expert_count;
    cfg[8] = t.config.expert_used_count;
    *rope = t.config.rope_freq_base;
    off[n++] = OFF(t.weights.token_embedding_table);
    off[n++] = OFF(t.weights.rms_final_weight);
    off[n++] = OFF(t.weights.wcls);
    types[m++] = t.weights.token_embd_type;
    types[m++] = t.weights.wcls_type;
    *row_bytes = t.weights.token_embd_row_bytes;
    for (l = 0; l < t.config.n_layers; l++) {
        off[n++] = OFF(t.weights.rms_att_weight[l]);
        off[n++] = OFF(t.weights.rms_ffn_weight[l]);
        off[n++] = OFF(t.weights.wq[l]);
        off[n++] = OFF(t.weights.wk[l]);
        off[n++] = OFF(t.weights.wv[l]);
        off[n++] = OFF(t.weights.wo[l]);
        off[n++] = t.config.expert_count > 0 ? OFF(t.weights.ffn_gate_inp[l]) : -1;
        types[m++] = t.weights.wq_type[l];
        types[m++] = t.weights.wk_type[l];
        types[m++] = t.weights.wv_type[l];
        types[m++] = t.weights.wo_type[l];
        if (t.config.expert_count > 0) {
            types[m++] = t.weights.exp_w1_type[l];
            types[m++] = t.weights.exp_w2_type[l];
            types[m++] = t.weights.exp_w3_type[l];
        } else { /* a dense model: w1 / w2 / w3 in the experts' places */
            types[m++] = t.weights.w1_type[l];
            types[m++] = t.weights.w2_type[l];
            types[m++] = t.weights.w3_type[l];
        }
    }
    for (l = 0; l < t.config.n_layers; l++) {
        if (t.config.expert_count == 0) {
            off[n++] = OFF(t.weights.w1[l]);
            off[n++] = OFF(t.weights.w2[l]);
            off[n++] = OFF(t.weights.w3[l]);
        }
        for (e = 0; e < t.config.expert_count; e++) {
            off[n++] = OFF(t.weights.expert_w1[l][e]);
            off[n++] = OFF(t.weights.expert_w2[l][e]);
            off[n++] = OFF(t.weights.expert_w3[l][e]);
        }
    }
#undef OFF
    free_transformer(&t);
    return n;
}
