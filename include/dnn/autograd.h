/* autograd.h -- only the grad-mode switch generation uses (reference
 * include/autograd.h:16-20, src/autograd.c:11-25); backward is not built here. */
#ifndef DNN_AUTOGRAD_H
#define DNN_AUTOGRAD_H

typedef struct { int _prev; } dnn_grad_ctx;
dnn_grad_ctx dnn_no_grad_enter(void);
void         dnn_no_grad_exit(dnn_grad_ctx ctx);
int          dnn_grad_enabled(void);

#endif
