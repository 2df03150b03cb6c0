/* oracle_main.c -- drives the oracle (oracle/dnn_oracle.c) from C so it can be
 * built with AddressSanitizer / UndefinedBehaviorSanitizer
 * (tests/test_sanitizers.py): a C1 model (synthetic init, seed 1), greedy
 * generation from the given prompt with the KV cache, and the no-cache
 * forward over the result; prints the ids as JSON.
 *
 *   oracle_main <new> <prompt ids...> */
#include "dnn_oracle.h"
#include <stdio.h>
#include <stdlib.h>

int main(int argc, char **argv) {
    if (argc < 3) return 2;
    const int NEW = atoi(argv[1]), P = argc - 2;
    int *prompt = malloc(sizeof(int) * (size_t)P), *out = malloc(sizeof(int) * (size_t)(P + NEW));
    for (int i = 0; i < P; i++) prompt[i] = atoi(argv[2 + i]);
    orc_cfg cfg = {128, 256, 4, 4, 64, 683, 256, 10000.0f};
    orc_model *m = orc_model_create(&cfg);
    orc_model_init_create(m, 1);
    orc_model_init_synthetic(m, 0.02f);
    orc_model_rope(m, cfg.max_seq, cfg.rope_base);
    const int n = orc_generate(m, prompt, P, NEW, -1, out, NULL);
    float *lg = malloc(sizeof(float) * (size_t)n * cfg.V);
    orc_forward_full(m, out, n, lg);
    int agree = 1;            /* the no-cache forward's argmax at the last prompt row */
    agree &= orc_argmax(lg + (size_t)(P - 1) * cfg.V, cfg.V) == out[P];
    printf("{\"tokens\": [");
    for (int i = 0; i < n; i++) printf("%s%d", i ? ", " : "", out[i]);
    printf("], \"nocache_agrees\": %d}\n", agree);
    free(lg); free(out); free(prompt);
    orc_model_free(m);
    return 0;
}
