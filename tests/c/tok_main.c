/* tok_main.c -- a caller of the reference's byte tokenizer API (tokenizer.h)
 * using only its declarations: built against the reference by
 * tests/golden/make_golden.sh (it writes tests/golden/data/tokenizer.json) and
 * against include/dnn by tests/test_host_api.py.  Prints one JSON object. */
#include "dnn.h"
#include "tokenizer.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void ids_json(const char *key, const int *ids, int n, int last) {
    printf("\"%s\": [", key);
    for (int i = 0; i < n; i++) printf("%s%d", i ? "," : "", ids[i]);
    printf("]%s", last ? "" : ", ");
}

static void str_json(const char *key, const char *s, int last) {
    printf("\"%s\": [", key);
    for (int i = 0; s[i]; i++) printf("%s%d", i ? "," : "", (unsigned char)s[i]);
    printf("]%s", last ? "" : ", ");
}

int main(void) {
    dnn_ctx ctx;
    if (dnn_ctx_init(&ctx, 1 << 20, 1 << 20, 1 << 20)) return 1;
    tokenizer d = tokenizer_default(), c = tokenizer_with_chat_template();
    tokenizer x = tokenizer_with_specials(NULL, "</s>", NULL);
    const char *t1 = "Hello, world!\n\xc3\xa9\x7f\x01";
    const char *t2 = "<|im_start|>user hi<|im_end|><|pad|>x<|im_start|";
    const char *t3 = "a</s>b</s</s>";
    int n1, n2, n3, n4, nz;
    int *e1 = tokenizer_encode(ctx.data, &d, t1, &n1);
    int *e2 = tokenizer_encode(ctx.data, &c, t2, &n2);
    int *e2d = tokenizer_encode(ctx.data, &d, t2, &n4);
    int *e3 = tokenizer_encode(ctx.data, &x, t3, &n3);
    int *ez = tokenizer_encode(ctx.data, &d, "", &nz);
    const int raw[] = {257, 72, 105, 258, 259, 260, 300, -5, 255, 0, 65, 256, 258};
    char *s1 = tokenizer_decode(&d, raw, (int)(sizeof raw / sizeof raw[0]));
    char *s2 = tokenizer_decode(&c, e2, n2);
    char *s0 = tokenizer_decode(&d, NULL, 0);
    tensor *tt = tokenizer_text_to_tensor(ctx.data, &c, t2);
    char *s3 = tokenizer_tensor_to_text(&c, tt);
    printf("{");
    ids_json("enc_default", e1, n1, 0);
    ids_json("enc_chat", e2, n2, 0);
    ids_json("enc_chat_as_default", e2d, n4, 0);
    ids_json("enc_eos_only", e3, n3, 0);
    printf("\"enc_empty\": [%d, %d], ", nz, ez == NULL);
    str_json("dec_raw", s1, 0);
    str_json("dec_chat", s2, 0);
    str_json("dec_empty", s0, 0);
    printf("\"tensor_shape\": [%d, %d], ", tt->shape[0], tt->shape[1]);
    str_json("tensor_text", s3, 1);
    printf("}\n");
    free(s1); free(s2); free(s0); free(s3);
    dnn_ctx_destroy(&ctx);
    return 0;
}
