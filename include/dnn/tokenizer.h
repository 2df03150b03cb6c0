/* tokenizer.h -- the byte-level tokenizer (reference include/tokenizer.h): ids
 * 0-255 are the byte values, 257-260 the special tokens; generation stops on
 * TOKENIZER_EOS_ID.  Host code (text <-> ids is no device work). */
#ifndef DNN_TOKENIZER_H
#define DNN_TOKENIZER_H
#include "tensor.h"

#define TOKENIZER_VOCAB_SIZE  261
#define TOKENIZER_BOS_ID      257
#define TOKENIZER_EOS_ID      258
#define TOKENIZER_PAD_ID      259
#define TOKENIZER_UNK_ID      260

/* Binary dataset header (reference tokenizer.h:31-45): magic, version,
 * vocab_size, num_sequences, seq_len, then reserved bytes up to 64, then
 * num_sequences x seq_len int32 ids. */
#define TOKENIZER_DATA_MAGIC       0x444E4E44  /* "DNND" */
#define TOKENIZER_DATA_VERSION     1
#define TOKENIZER_DATA_HEADER_SIZE 64

typedef struct {
    int  bos_id;
    int  eos_id;
    int  pad_id;
    int  unk_id;
    const char *bos_str;   /* optional special-token strings, e.g. "<|im_start|>" */
    const char *eos_str;
    const char *pad_str;
    int  bos_len;          /* strlen of each, 0 when NULL */
    int  eos_len;
    int  pad_len;
} tokenizer;

/* BOS 257, EOS 258, PAD 259, UNK 260, no special strings. */
tokenizer tokenizer_default(void);
/* The chat template's strings "<|im_start|>", "<|im_end|>", "<|pad|>". */
tokenizer tokenizer_with_chat_template(void);
/* Explicit special strings (NULL: none). */
tokenizer tokenizer_with_specials(const char *bos_str, const char *eos_str, const char *pad_str);

/* text -> BOS, one id per byte (a special string's occurrence -> its id), EOS;
 * from the data pool, *len ids; NULL and *len = 0 for empty text. */
int *tokenizer_encode(struct mem_pool *data_pool, tokenizer *tok, const char *text, int *len);
/* ids -> text (malloc'd, caller frees): BOS/EOS/PAD dropped, ids outside
 * [0, 256) become '?'; "" for no ids. */
char *tokenizer_decode(tokenizer *tok, const int *ids, int len);
/* text -> an int tensor [1, N] in the data pool (NULL for empty text). */
tensor *tokenizer_text_to_tensor(struct mem_pool *data_pool, tokenizer *tok, const char *text);
/* the ids of an int tensor -> text (malloc'd). */
char *tokenizer_tensor_to_text(tokenizer *tok, const tensor *t);

#endif
