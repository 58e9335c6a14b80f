// The ggml backend add-on's internals shared between the policy (what the
// scheduler may hand us) and the executor (graph_compute).
#pragma once

#include <string>
#include <unordered_set>

#include "zest_ggml.h"

namespace zest {

// How the backend runs, decided once at registration (src/ggml-zest.cpp:91-118):
// the GPU opens, is a gfx950, and gets the registration known-answer multiply
// right; otherwise no device is offered. There is no CPU path.
enum class run_mode { off, gpu };
run_mode mode();
int device_index();
// GGML_XDNA_PLAN_ONLY=1: the device is offered for planning only (no GPU is
// opened, no memory reported, every graph_compute fails).
bool plan_only();

// Set when the GPU path fails during a graph (a kernel error, non-finite
// results, an injected failure): from then on the backend claims nothing
// (src/ggml-zest.cpp:123-130).
bool broken();
void mark_broken(const std::string & why);

// Settings (docs/technical-guide.md:562-574 of the reference; same names).
int64_t min_batch();   // GGML_XDNA_MIN_BATCH, default 1024
int64_t min_mflop();   // GGML_XDNA_MIN_MFLOP, default 256
bool blocks();         // GGML_XDNA_BLOCKS, default on: claim the small ops next to our matmuls
bool trace();          // GGML_XDNA_TRACE

// The gate (src/ggml-zest.cpp:1160-1226).
bool supports_op(const ggml_tensor * op);
bool claim_mul_mat(const ggml_tensor * op);
bool is_weight(const ggml_tensor * w);
bool exec_supports(const ggml_tensor * op);
const ggml_tensor * exec_param(const ggml_tensor * op);
// Whether one GEMM launch addresses an M x K activation operand, a K x N
// weight's cache entry, and output bands of 256 rows of N floats, each under
// 2 GiB (the kernels' buffer ranges); the library cuts a taller output into
// bands itself.
bool gemm_shape_fits(int64_t M, int64_t K, int64_t N);

// Reader tracking (src/ggml-zest.cpp:1082-1109): every op the scheduler asks
// about records its inputs' readers; a result is needed outside a graph piece
// when a reader outside it exists, it is a graph output, or it was never seen.
void note_readers(const ggml_tensor * op);
bool read_outside(const ggml_tensor * t, const std::unordered_set<const ggml_tensor *> & in_piece);
// Changes whenever a new reader is recorded (what read_outside answers may change with it).
uint64_t readers_epoch();

// The HBM budget for weight-cache entries (src/ggml-zest.cpp:429-564).
double copy_bytes(int64_t K, int64_t N);
bool budget_takes(const ggml_tensor * w);
void budget_context_added();
void budget_context_freed();
void budget_report();

// Model notes said once (src/ggml-zest.cpp:570-637).
void note_model(const ggml_tensor * op);
void say_notes();

} // namespace zest
