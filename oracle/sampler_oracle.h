/* sampler_oracle.h -- CPU restatement of gguf-rs-cli src/sampler.rs.
 * TEST INFRASTRUCTURE ONLY (parity checker); never linked into the product. */
#ifndef SAMPLER_ORACLE_H
#define SAMPLER_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_ERR_NAN   (-3)
#define ORACLE_ERR_EMPTY (-2)
#define ORACLE_ERR_NOMEM (-6)

typedef struct { float temperature; uint32_t top_k; float top_p; float rep_penalty; } oracle_params;

typedef struct {
    uint32_t *idx; float *p; size_t cap; /* caller buffers for post-softmax probs */
    size_t n_kept; size_t cut; float sum; float s2; float r; float q_last;
} oracle_detail;

void oracle_set_seed(uint64_t s);
uint64_t oracle_get_seed(void);
float oracle_lcg_draw(uint64_t *state);
void oracle_apply_rep_penalty(float *l, size_t n, const uint32_t *recent, size_t w, float penalty);
int64_t oracle_sample_ex(float *logits, size_t V, float temperature, size_t top_k, float top_p,
                         float rep_penalty, const uint32_t *recent, size_t W, float r,
                         uint64_t *draw_state, int fast_topk, oracle_detail *det);
int64_t oracle_sample(float *logits, size_t V, float temperature, size_t top_k, float top_p,
                      float rep_penalty, const uint32_t *recent, size_t W);
int oracle_sample_batch(const float *logits, size_t B, size_t V, size_t ld,
                        const oracle_params *params, const uint32_t *recent, size_t ld_recent,
                        const uint32_t *recent_len, size_t W, const float *u, int64_t *tokens,
                        int nthreads, int fast_topk);
int oracle_decode_trace(const float *logits, size_t steps, size_t V, float temperature,
                        size_t top_k, float top_p, float rep_penalty, size_t window,
                        const uint32_t *init_recent, size_t init_len, uint64_t seed,
                        int64_t *tokens, int fast_topk);
float oracle_synth_logit(uint64_t seed, uint64_t counter, float sigma);
void oracle_synth_logits(float *out, size_t n, uint64_t seed, uint64_t counter0, float sigma);
int oracle_device_loop(size_t B, size_t V, size_t steps, uint64_t seed, float sigma,
                       const oracle_params *p, uint32_t *window, size_t W, const float *u,
                       int64_t *tokens, int nthreads, int fast_topk);
double oracle_now(void);

#ifdef __cplusplus
}
#endif
#endif
