/*
 * ggml-zest.h — the public registration of the MI355X ggml backend add-on,
 * with the reference's names (include/ggml-zest.h:10-13 of Cyronius/ggml-xdna):
 * llama.cpp loads libggml-zest.so with ggml_backend_load and finds one device,
 * "XDNA0", that takes large-batch prompt MUL_MATs (and the small ops between
 * them) and runs them on the GPU with bfp16 operands.
 */
#ifndef GGML_ZEST_H
#define GGML_ZEST_H

#include "ggml_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_XDNA_NAME "XDNA"         /* the backend (registry) name */
#define GGML_XDNA_DEVICE_NAME "XDNA0" /* the device, as -dev names it */

/* The registry object (src/ggml-zest.cpp:1294-1301). */
GGML_BACKEND_API ggml_backend_reg_t ggml_backend_xdna_reg(void);

/* The dynamic-loading entry points llama.cpp's ggml_backend_load looks up
 * (GGML_BACKEND_DL_IMPL / GGML_BACKEND_DL_SCORE_IMPL, src/ggml-zest.cpp:1314-1319). */
GGML_BACKEND_API ggml_backend_reg_t ggml_backend_init(void);
GGML_BACKEND_API int ggml_backend_score(void);

#ifdef __cplusplus
}
#endif
#endif
