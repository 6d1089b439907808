/*
 * Test infrastructure: exposes the reference driver's token sampler, which is
 * static in src/runtime_main.c (sample_token, :213-248, and the LCG state of
 * :205-211), by compiling that file here with its main renamed.  Built only
 * by `make -C oracle ref` where the reference tree exists, into _ref/.
 */
#define main ec_ref_runtime_main
#include "runtime_main.c"
#undef main

int ref_sample_token(const float *logits, int vocab, float temp, int top_k)
{
    return sample_token(logits, vocab, temp, top_k);
}

void ref_rng_set(unsigned long long s) { rng_state = (unsigned long)s; }

unsigned long long ref_rng_get(void) { return (unsigned long long)rng_state; }
