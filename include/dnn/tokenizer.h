/* tokenizer.h -- the byte tokenizer's special ids (reference include/tokenizer.h:22-26);
 * generation stops on TOKENIZER_EOS_ID. */
#ifndef DNN_TOKENIZER_H
#define DNN_TOKENIZER_H

#define TOKENIZER_VOCAB_SIZE  261
#define TOKENIZER_BOS_ID      257
#define TOKENIZER_EOS_ID      258
#define TOKENIZER_PAD_ID      259
#define TOKENIZER_UNK_ID      260

#endif
