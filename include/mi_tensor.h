/*
 * mi_tensor.h -- the engine's tensor/graph layout, restated so that host code
 * built against this repository can exchange tensors with the mini-infer CPU
 * engine without any conversion.
 *
 * Every enum value, field, field order and field type below is chosen to be
 * ABI-identical to the reference engine:
 *   - element types       src/tensor.h:20-34
 *   - op codes            src/tensor.h:49-99 (ATTN_QK = 16, ATTN_KQV = 17,
 *                         SOFTMAX = 7, CPY = 10)
 *   - tensor flags        src/tensor.h:112-117
 *   - struct mi_tensor    src/tensor.h:122-160
 *   - struct mi_cgraph    src/graph.h:19-47
 * A static layout check (mi_hip_abi_layout in mi_hip_attn.h) lets a caller
 * assert at run time that both sides agree on sizeof/offsetof.
 *
 * The header is plain C so it can be used from C, C++ and ctypes alike.
 */
#ifndef MI_TENSOR_H
#define MI_TENSOR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_MAX_DIMS 4
#define MI_MAX_SRC 2
#define MI_MAX_OP_PARAMS 8
#define MI_MAX_NAME 64

/* Element type tags (src/tensor.h:20-34). */
typedef enum mi_type {
  MI_TYPE_F32 = 0,
  MI_TYPE_F16 = 1,
  MI_TYPE_Q8_0 = 2,
  MI_TYPE_I32 = 3,
  MI_TYPE_Q8_0_ACT = 4,
  MI_TYPE_COUNT = 5
} mi_type;

/* Graph op codes (src/tensor.h:49-102). Numeric values are part of the ABI. */
typedef enum mi_op {
  MI_OP_NONE = 0,
  MI_OP_GET_ROWS = 1,
  MI_OP_RMS_NORM = 2,
  MI_OP_MUL = 3,
  MI_OP_ADD = 4,
  MI_OP_MUL_MAT = 5,
  MI_OP_ROPE = 6,
  MI_OP_SOFTMAX = 7,
  MI_OP_SILU = 8,
  MI_OP_SCALE = 9,
  MI_OP_CPY = 10,
  MI_OP_QUANTIZE_Q8_0 = 11,
  MI_OP_RESHAPE = 12,
  MI_OP_VIEW = 13,
  MI_OP_PERMUTE = 14,
  MI_OP_TRANSPOSE = 15,
  MI_OP_ATTN_QK = 16,
  MI_OP_ATTN_KQV = 17,
  MI_OP_COUNT = 18
} mi_op;

/* Tensor flags (src/tensor.h:112-117). */
#define MI_TENSOR_FLAG_WEIGHT (1u << 0)
#define MI_TENSOR_FLAG_INPUT (1u << 1)
#define MI_TENSOR_FLAG_OUTPUT (1u << 2)
#define MI_TENSOR_FLAG_KV (1u << 3)

/*
 * N-d array descriptor and graph node. ne[0] is the innermost dimension;
 * nb[k] is the byte stride of dimension k. Element (i0,i1,i2,i3) lives at
 * data + i0*nb[0] + i1*nb[1] + i2*nb[2] + i3*nb[3].
 */
typedef struct mi_tensor {
  mi_type type;
  int64_t ne[MI_MAX_DIMS];
  size_t nb[MI_MAX_DIMS];
  mi_op op;
  int32_t op_params[MI_MAX_OP_PARAMS]; /* i32 values, or f32 bit patterns */
  struct mi_tensor* src[MI_MAX_SRC];
  void* data;
  struct mi_tensor* view_src; /* storage owner when this tensor is a view */
  size_t view_offs;
  int32_t n_children;
  uint32_t flags;
  char name[MI_MAX_NAME];
  void* extra; /* rewritten by the engine's allocator every step: never a handle */
} mi_tensor;

/* Topologically sorted graph (src/graph.h:19-47). */
typedef struct mi_cgraph {
  mi_tensor** nodes;
  int n_nodes;
  mi_tensor** leafs;
  int n_leafs;
  mi_tensor** exec_nodes; /* nodes minus the pure-view ops */
  int n_exec_nodes;
  int capacity;
} mi_cgraph;

/* op_params slot access, memcpy semantics (src/ops_cpu.cpp:84-99). */
static inline int32_t mi_tensor_param_i32(const mi_tensor* t, int slot) {
  return t->op_params[slot];
}
static inline float mi_tensor_param_f32(const mi_tensor* t, int slot) {
  union {
    int32_t i;
    float f;
  } u;
  u.i = t->op_params[slot];
  return u.f;
}

#ifdef __cplusplus
}
#endif

#endif /* MI_TENSOR_H */
