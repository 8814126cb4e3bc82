// rt.h — internals shared by the runtime's translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdarg>
#include <string>
#include "../kernels/args.h"
#include "../../../include/cajeta_mi355x.h"

namespace cj {

int fail(int code, const char *fmt, ...);
const char *last_error();
const char *last_launch();   // the name of the last kernel launched on this thread
void launch_names_reset();    // start a new record of the kernels launched on this thread
const char *launch_names();   // their distinct names in first-launch order, " + "-joined
uint64_t launch_count();     // launches made so far

bool ready();
hipStream_t stream();
int device_cus();

// The allocation containing [p, p + bytes), or false.
bool in_buffer(const void *p, int64_t bytes);
void *dptr(int64_t h);

// Launch `name` from kernels.hsaco with one argument block.
int launch_raw(const char *name, uint32_t grid, uint32_t block, uint32_t lds, const void *args, size_t size,
               uint32_t grid_y = 1);
template <class A>
int launch(const char *name, uint32_t grid, uint32_t block, uint32_t lds, const A &a) {
    return launch_raw(name, grid, block, lds, &a, sizeof(A));
}
template <class A>
int launch2(const char *name, uint32_t grid_x, uint32_t grid_y, uint32_t block, uint32_t lds, const A &a) {
    return launch_raw(name, grid_x, block, lds, &a, sizeof(A), grid_y);
}
bool has_kernel(const char *name);
bool q4k_unrolled();

// GEMV planning shared by the launch seam and the engine.
struct GemvPlan {
    std::string kernel;
    int rows_per_wg = 0;
    uint32_t grid = 0;
    uint32_t per_copy = 0;   // workgroups per expert copy (MoE indirection)
    uint32_t lds = 0;
};
int64_t prepared_row_bytes(int type, int64_t cols);
bool is_f32_act(int type);
bool gemv_supported(int type, int64_t cols);
// Kernel, rows per workgroup (`target` rounded to what one pass of the
// workgroup covers, at most 256; 0 = one pass), grid and LDS of a GEMV.
GemvPlan plan_gemv(int type, int64_t rows, int64_t cols, int target, int pro, int epi);
int run_gemv(const cj_gemv_args &a, const GemvPlan &p);
// The batched mat-mat on the int8 matrix cores (Q8_0, Q4_K): a.batch columns
// of packed activations a.xp (a.xp_stride bytes apart) into a.y (a.y_stride
// floats apart); STORE or ACCUM epilogue.
bool gemm_supported(int type);
int run_gemm(const cj_gemv_args &a);

// Device memory owned by the runtime itself (not through the handle table's
// public free): allocation + registration for the extent checks.
void *dev_alloc(size_t bytes);
void dev_free(void *p);

}  // namespace cj

#define CJ_HIP(x)                                                                         \
    do {                                                                                  \
        hipError_t e__ = (x);                                                             \
        if (e__ != hipSuccess) return cj::fail(CJ_ERR_HIP, "%s: %s", #x, hipGetErrorString(e__)); \
    } while (0)
