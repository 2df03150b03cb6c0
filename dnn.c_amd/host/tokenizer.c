/* tokenizer.c -- the byte-level tokenizer (reference src/tokenizer.c:9-182):
 * every byte is its own id, special-token strings (when set) are matched at
 * each position in the order BOS, EOS, PAD before falling back to the byte;
 * encode brackets the ids with BOS and EOS, decode drops BOS/EOS/PAD and maps
 * anything outside the byte range to '?'. */
#include "dnn/tokenizer.h"
#include <assert.h>
#include <stdlib.h>
#include <string.h>

tokenizer tokenizer_default(void) {
    tokenizer t;
    memset(&t, 0, sizeof t);
    t.bos_id = TOKENIZER_BOS_ID;
    t.eos_id = TOKENIZER_EOS_ID;
    t.pad_id = TOKENIZER_PAD_ID;
    t.unk_id = TOKENIZER_UNK_ID;
    return t;
}

tokenizer tokenizer_with_specials(const char *bos_str, const char *eos_str, const char *pad_str) {
    tokenizer t = tokenizer_default();
    t.bos_str = bos_str;
    t.eos_str = eos_str;
    t.pad_str = pad_str;
    t.bos_len = bos_str ? (int)strlen(bos_str) : 0;
    t.eos_len = eos_str ? (int)strlen(eos_str) : 0;
    t.pad_len = pad_str ? (int)strlen(pad_str) : 0;
    return t;
}

tokenizer tokenizer_with_chat_template(void) {
    return tokenizer_with_specials("<|im_start|>", "<|im_end|>", "<|pad|>");
}

/* The special id whose string starts at text[pos] (first of BOS, EOS, PAD
 * that fits and matches), its length in *n; -1 when none does. */
static int special_at(const tokenizer *t, const char *text, int pos, int text_len, int *n) {
    const char *str[3] = {t->bos_str, t->eos_str, t->pad_str};
    const int len[3] = {t->bos_len, t->eos_len, t->pad_len};
    const int id[3] = {t->bos_id, t->eos_id, t->pad_id};
    for (int k = 0; k < 3; k++) {
        if (!str[k] || len[k] <= 0 || pos + len[k] > text_len) continue;
        if (memcmp(text + pos, str[k], (size_t)len[k]) == 0) {
            *n = len[k];
            return id[k];
        }
    }
    return -1;
}

int *tokenizer_encode(struct mem_pool *data_pool, tokenizer *tok, const char *text, int *len) {
    assert(tok && len);
    if (!text || !text[0]) {
        *len = 0;
        return NULL;
    }
    const int n_text = (int)strlen(text);
    int *ids = _mem_pool_alloc(data_pool, sizeof(int) * (size_t)(n_text + 2), NULL);
    int n = 0;
    ids[n++] = tok->bos_id;
    for (int i = 0; i < n_text;) {
        int step = 1;
        const int sp = special_at(tok, text, i, n_text, &step);
        ids[n++] = sp >= 0 ? sp : (int)(unsigned char)text[i];
        i += sp >= 0 ? step : 1;
    }
    ids[n++] = tok->eos_id;
    *len = n;
    return ids;
}

char *tokenizer_decode(tokenizer *tok, const int *ids, int len) {
    assert(tok);
    if (!ids || len <= 0) {
        char *e = malloc(1);
        if (e) e[0] = '\0';
        return e;
    }
    char *s = malloc((size_t)len + 1);
    if (!s) return NULL;
    int n = 0;
    for (int i = 0; i < len; i++) {
        const int id = ids[i];
        if (id == tok->bos_id || id == tok->eos_id || id == tok->pad_id) continue;
        s[n++] = id >= 0 && id < 256 ? (char)(unsigned char)id : '?';
    }
    s[n] = '\0';
    return s;
}

tensor *tokenizer_text_to_tensor(struct mem_pool *data_pool, tokenizer *tok, const char *text) {
    int n = 0;
    int *ids = tokenizer_encode(data_pool, tok, text, &n);
    if (!ids || n <= 0) return NULL;
    tensor *t = tensor_zeros_data(data_pool, 2, (int[]){1, n});
    memcpy(t->data, ids, sizeof(int) * (size_t)n);
    return t;
}

char *tokenizer_tensor_to_text(tokenizer *tok, const tensor *t) {
    if (!t || tensor_numel(t) == 0) return tokenizer_decode(tok, NULL, 0);
    return tokenizer_decode(tok, (const int *)t->data + t->offset, tensor_numel(t));
}
