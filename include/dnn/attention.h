/* attention.h -- attention modes (reference include/attention.h:22-25). */
#ifndef DNN_ATTENTION_H
#define DNN_ATTENTION_H

typedef enum attention_mode {
    ATTENTION_CAUSAL = 0,
    ATTENTION_PREFIX_LM = 1
} attention_mode;

#endif
