/* autograd.c -- thread-local grad mode (reference src/autograd.c:11-25). */
#include "dnn/autograd.h"

static _Thread_local int g_grad_enabled = 1;

dnn_grad_ctx dnn_no_grad_enter(void) {
    dnn_grad_ctx c = {g_grad_enabled};
    g_grad_enabled = 0;
    return c;
}

void dnn_no_grad_exit(dnn_grad_ctx ctx) { g_grad_enabled = ctx._prev; }
int  dnn_grad_enabled(void) { return g_grad_enabled; }
