/* dnn.h -- umbrella header of the MI355X decode library (reference include/dnn.h). */
#ifndef DNN_H
#define DNN_H
#include "pool.h"
#include "context.h"
#include "tensor.h"
#include "rng.h"
#include "autograd.h"
#include "module.h"
#include "nn.h"
#include "ops.h"
#include "norm.h"
#include "multihead.h"
#include "attention.h"
#include "rope.h"
#include "tokenizer.h"
#include "transformer.h"
#include "gpt.h"
#include "vlm.h"
#endif
