// runtime.cpp — the C-ABI runtime: device + stream, the kernels.hsaco
// module and its registry, the device-buffer table behind every extent
// check, graphs and events, and the launch seam (one validated launch per
// reference *LaunchNoSync wrapper).
#include "rt.h"
#include <dlfcn.h>
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

// The scratch of cj_argmax_row_noalloc: the per-workgroup (value, index)
// partials and the ticket counter of the argmax kernel, in one file-scope
// device array so that entry point allocates nothing. Every GPU the library
// runs on holds its own copy until the process ends; host code reaches it
// only through the per-device address hipGetSymbolAddress returns (the
// array's name is a host-side stand-in, not a device address).
#define CJ_NOALLOC_ARGMAX_MAX (1 << 22)                    // values a row may hold
#define CJ_NOALLOC_GROUPS (CJ_NOALLOC_ARGMAX_MAX / 1024)   // workgroups of 1024 values
static __device__ __align__(256) uint8_t scratch[CJ_NOALLOC_GROUPS * 8 + 256];

namespace cj {

namespace {
struct Ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    hipModule_t module = nullptr;
    std::unordered_map<std::string, hipFunction_t> fns;
    std::map<uintptr_t, size_t> allocs;
    std::mutex mu;
    int cus = 0;
    int64_t hbm = 0;
    int64_t lds = 0;
    std::map<int, void *> scratch_at;   // device → address of `scratch` on it
};
Ctx g;
thread_local std::string g_err;
thread_local std::string g_last_launch;
thread_local std::string g_launch_names;    // distinct names since launch_names_reset, " + "-joined
thread_local bool g_naming = false;         // recording them (until launch_names)
uint64_t g_launches = 0;   // launches made (the timing seam checks a kind launched something)

// The reference's kernel names (KernelCap.nameOf, model/KernelCap.cajeta:100-140
// and the launch sites) answered by the kernels of this code object. A name
// is listed only where the kernel here computes what the named one computes
// and a parity test covers it; the reference's CPU-backend kernel names and
// the fused MoE id kernels (whose combine and Q4_K experts this backend does
// not serve) are answered "no".
const std::unordered_map<std::string, std::string> &name_map() {
    static const std::unordered_map<std::string, std::string> m = {
        {"q4kQ8WaveMatVecKernel", "cj_gemv_q4k_cs_b16"},
        {"q6kQ8WaveMatVecKernel", "cj_gemv_q6k_l64"},
        {"q80Q8WaveMatVecKernel", "cj_gemv_q80_l64"},
        {"q40F32WaveMatVecKernel", "cj_gemv_q40b_r4"},
        {"mxfp4MatVecKernel", "cj_gemv_mxfp4"},
        {"mxfp4MatVecKernelCoopQ8", "cj_gemv_mxq8_s_k3_r4"},
        {"q8kPackKernel", "cj_pack"},
        {"q8kPack32Kernel", "cj_pack"},
        {"rmsnormPackRowF32", "cj_pack"},
        {"rmsnormRowF32", "cj_pack"},
        {"gluPackF32", "cj_glu"},
        {"gluF32", "cj_glu"},
        {"addF32", "cj_add"},
        {"qkPrepKernel", "cj_qkprep"},
        {"attnFlashDecodeGqa4Kernel", "cj_attn_split_h128_g4"},
        {"attnFlashDecodeGqa8Kernel", "cj_attn_split_h128_g8"},
        {"attnScoreKernel", "cj_attn_scores_h64"},
        {"attnCombineKernel", "cj_attn_combine_h64"},
        {"attnReducePackQ8Kernel", "cj_attn_merge"},
        {"attnReducePackQ8BatchKernel", "cj_attn_merge_rows"},
        {"attnFlashDecodeGqa4BatchKernel", "cj_attn_split_rows_h128_g4"},
        {"argmaxRowKernel", "cj_argmax"},
        {"embedRowQ4kKernel", "cj_embed"},
        {"embedRowQ6kKernel", "cj_embed"},
        {"embedRowQ80Kernel", "cj_embed"},
        {"gatherRowsF32Kernel", "cj_embed"},
        {"routerTopKKernel", "cj_router_topk"},
        {"q4kQ8WaveMatVecColsKernel", "cj_gemm_sk_q4k_n1"},
    };
    return m;
}

std::string module_path() {
    if (const char *e = getenv("CJ_KERNELS_HSACO")) return e;
    Dl_info info;
    if (dladdr((void *)&cj_init, &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        size_t s = p.rfind('/');
        return (s == std::string::npos ? std::string(".") : p.substr(0, s)) + "/kernels.hsaco";
    }
    return "kernels.hsaco";
}
}  // namespace

int fail(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
const char *last_error() { return g_err.c_str(); }
const char *last_launch() { return g_last_launch.c_str(); }
void launch_names_reset() { g_launch_names.clear(); g_naming = true; }
const char *launch_names() { g_naming = false; return g_launch_names.c_str(); }
bool ready() { return g.module != nullptr; }
hipStream_t stream() { return g.stream; }
int device_cus() { return g.cus; }

bool in_buffer(const void *p, int64_t bytes) {
    if (bytes < 0) return false;
    std::lock_guard<std::mutex> lk(g.mu);
    uintptr_t a = (uintptr_t)p;
    auto it = g.allocs.upper_bound(a);
    if (it == g.allocs.begin()) return false;
    --it;
    return a >= it->first && a + (uintptr_t)bytes <= it->first + it->second;
}
void *dptr(int64_t h) { return (void *)(uintptr_t)h; }

void *dev_alloc(size_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lk(g.mu);
    g.allocs[(uintptr_t)p] = bytes ? bytes : 16;
    return p;
}
void dev_free(void *p) {
    if (!p) return;
    {
        std::lock_guard<std::mutex> lk(g.mu);
        g.allocs.erase((uintptr_t)p);
    }
    (void)hipFree(p);
}

bool has_kernel(const char *name) { return g.fns.count(name) != 0; }

// Whether Q4_K GEMVs take the fully unrolled forms where built
// (CJ_Q4K_UNROLL=0 keeps the runtime-loop forms, for comparisons).
bool q4k_unrolled() {
    static const bool on = [] { const char *e = getenv("CJ_Q4K_UNROLL"); return !e || strcmp(e, "0") != 0; }();
    return on;
}

// The address of `scratch` on the current device, resolved once per device
// with that device current; its counter word is zeroed then (the argmax
// kernel leaves it zero after every launch).
int scratch_here(void **out) {
    int dev = -1;
    CJ_HIP(hipGetDevice(&dev));
    auto it = g.scratch_at.find(dev);
    if (it != g.scratch_at.end()) { *out = it->second; return CJ_OK; }
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(CJ_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    CJ_HIP(hipMemset(p, 0, sizeof(scratch)));
    CJ_HIP(hipDeviceSynchronize());
    g.scratch_at[dev] = p;
    *out = p;
    return CJ_OK;
}

int launch_raw(const char *name, uint32_t grid, uint32_t block, uint32_t lds, const void *args, size_t size,
               uint32_t grid_y) {
    if (!ready()) return fail(CJ_ERR_STATE, "cj_init has not run");
    auto it = g.fns.find(name);
    if (it == g.fns.end()) return fail(CJ_ERR_NOKERNEL, "kernel %s is not in kernels.hsaco", name);
    if (grid == 0 || grid_y == 0) return CJ_OK;
    (void)size;
    // every kernel takes one argument, the struct: kernelParams[0] points at it
    void *params[] = {const_cast<void *>(args)};
    hipError_t e = hipModuleLaunchKernel(it->second, grid, grid_y, 1, block, 1, 1, lds, g.stream, params, nullptr);
    if (e != hipSuccess) return fail(CJ_ERR_HIP, "launch %s: %s", name, hipGetErrorString(e));
    g_last_launch = name;
    if (g_naming && (" + " + g_launch_names + " + ").find(" + " + std::string(name) + " + ") == std::string::npos)
        g_launch_names += (g_launch_names.empty() ? "" : " + ") + std::string(name);
    g_launches++;
    return CJ_OK;
}

uint64_t launch_count() { return g_launches; }

// ------------------------------------------------------------------ GEMV

bool is_f32_act(int type) { return type == CJ_Q4_0 || type == CJ_MXFP4 || type == CJ_F32; }

int64_t prepared_row_bytes(int type, int64_t cols) {
    auto pad16 = [](int64_t v) { return (v + 15) / 16 * 16; };
    switch (type) {
    case CJ_Q4_K: return cols % 256 ? -1 : cols / 256 * 144;
    case CJ_Q6_K: return cols % 256 ? -1 : cols / 256 * 208 + pad16(cols / 256 * 2);
    case CJ_Q8_0: return cols % 32 ? -1 : cols / 32 * 32 + pad16(cols / 32 * 2);
    case CJ_Q4_0: return cols % 32 ? -1 : cols / 32 * 16 + pad16(cols / 32 * 2);
    case CJ_MXFP4: return cols % 32 ? -1 : cols / 32 * 16 + pad16(cols / 32);
    case CJ_F32: return cols % 4 ? -1 : cols * 4;
    default: return -1;
    }
}

bool gemv_supported(int type, int64_t cols) {
    // the staged activation and the per-row terms stay within 64 KB of LDS;
    // the f32 rows are walked in whole 32-element blocks
    return prepared_row_bytes(type, cols) > 0 && cols <= (is_f32_act(type) ? 15360 : 16384) &&
           (type != CJ_F32 || cols % 32 == 0);
}

// Q4_K: LPR lanes a row (one lane a block), rows a workgroup in whole passes
// of 4·(64 / LPR), about rows / CUs of them so one wave of workgroups covers
// the matrix, bounded by one folding thread a row and by LDS (the staged
// pack at 336 bytes a block + 8 bytes of terms a row and block). The kernel
// is picked by the prologue (copied pack, f32 pack, RMSNorm + pack) and the
// activation width (up to 4096 columns, or up to 16384 without the norm).
GemvPlan plan_gemv_q4k(int64_t rows, int64_t cols, int pro, int epi) {
    GemvPlan p;
    const int64_t nb = cols / 256;
    // wide rows (the FFN down projection) take a row a wave
    const int lpr = nb > 32 && cols > 4096 ? 64 : nb >= 16 ? 16 : 8;
    const int64_t pass = 4 * (64 / lpr);
    // the RMSNorm prologue runs once a workgroup: round up (fewer, longer
    // workgroups); otherwise round down (every CU busy)
    const int64_t per_cu = rows / std::max(1, g.cus);
    int64_t R = pro == CJ_PRO_NORM_PACK ? (per_cu + pass - 1) / pass * pass : per_cu / pass * pass;
    const int64_t fixed = 3072 + nb * 336;
    const int64_t rmax = std::min<int64_t>((65536 - fixed) / (nb * 8), 256) / pass * pass;
    R = std::max<int64_t>(pass, std::min(R, rmax));
    const char pc = pro == CJ_PRO_PACKED ? 'c' : pro == CJ_PRO_PACK ? 'p' : pro == CJ_PRO_NORM_PACK ? 'n' : '?';
    const char ec = epi == CJ_EPI_STORE ? 's' : epi == CJ_EPI_ACCUM ? 'a' : epi == CJ_EPI_QKV_ROPE ? 'q'
                  : epi == CJ_EPI_GLU ? 'g' : epi == CJ_EPI_ARGMAX ? 'm' : '?';
    p.kernel = std::string("cj_gemv_q4k_") + pc + ec + (lpr == 64 ? "_b64" : lpr == 16 ? "_b16" : "_b8") + (cols > 4096 ? "_w" : "");
    // the fully unrolled form where one is built for this item count
    const int64_t K = (nb + lpr - 1) / lpr, items = (R / pass) * K;
    const std::string unrolled = p.kernel + "_i" + std::to_string(items);
    if (q4k_unrolled() && has_kernel(unrolled.c_str())) p.kernel = unrolled;
    p.rows_per_wg = (int)R;
    p.grid = (uint32_t)((rows + R - 1) / R);
    p.per_copy = p.grid;
    p.lds = (uint32_t)(fixed + R * nb * 8);
    return p;
}

GemvPlan plan_gemv(int type, int64_t rows, int64_t cols, int target, int pro, int epi) {
    if (type == CJ_Q4_K) return plan_gemv_q4k(rows, cols, pro, epi);
    GemvPlan p;
    if (type == CJ_MXFP4 && pro == CJ_PRO_MXQ8) {
        // RW rows a 32-lane half-wave (their 16-byte code loads in flight
        // together), 8·RW rows a workgroup: 32, or 16 for matrices of at
        // most 4096 rows (twice the workgroups); KB blocks a lane a sweep
        const int64_t nb = cols / 32;
        const int kb = (int)std::min<int64_t>(4, std::max<int64_t>(1, (nb + 31) / 32));
        const int rw = rows <= 4096 ? 2 : 4;
        const char ec = epi == CJ_EPI_STORE ? 's' : epi == CJ_EPI_ACCUM ? 'a' : epi == CJ_EPI_GLU ? 'g' : '?';
        p.kernel = std::string("cj_gemv_mxq8_") + ec + "_k" + std::to_string(kb) + "_r" + std::to_string(rw);
        p.rows_per_wg = 8 * rw;
        p.grid = (uint32_t)((rows + p.rows_per_wg - 1) / p.rows_per_wg);
        p.per_copy = p.grid;
        p.lds = 3072 + (uint32_t)((cols + 15) & ~15) + (uint32_t)((nb + 3) & ~3) * 4 + 32 * 4;
        return p;
    }
    const char *fam = type == CJ_Q4_K ? "cj_gemv_q4k" : type == CJ_Q6_K ? "cj_gemv_q6k" : type == CJ_Q8_0 ? "cj_gemv_q80"
                      : type == CJ_MXFP4 ? "cj_gemv_mxfp4" : "cj_gemv_f32";
    if (type == CJ_Q4_0) {
        // block-parallel: RW rows a wave, 4·RW a workgroup; 2 where 4 would
        // leave the matrix under two workgroups a CU
        const int rw = rows <= 8 * (int64_t)std::max(1, g.cus) * 2 ? 2 : 4;
        p.kernel = std::string("cj_gemv_q40b_r") + std::to_string(rw);
        p.rows_per_wg = 4 * rw;
        p.grid = (uint32_t)((rows + p.rows_per_wg - 1) / p.rows_per_wg);
        p.per_copy = p.grid;
        p.lds = 3072 + (uint32_t)((cols + 255) / 256 * 1024);
        return p;
    }
    if (is_f32_act(type)) {
        // 64 rows a workgroup, each summed in element order by one lane; 32
        // (six blocks a tile for the producers, half the tiles) where 64-row
        // workgroups would leave a quarter of the CUs idle. Measured: MXFP4
        // 11520×2880 22.7 → 19.8 µs at 32; a 14336×4096 chain 31 → 40 µs at 32
        // (1 for at most 64 rows — a router: every producer lane on one row,
        // a 2880-wide row in one tile, a workgroup a row)
        const int R = rows <= 64 ? 1 : rows <= 48 * (int64_t)std::max(1, g.cus) ? 32 : 64;
        p.kernel = std::string(fam) + (R == 32 ? "_r32" : R == 1 ? "_r1" : "");
        p.rows_per_wg = R;
        p.grid = (uint32_t)((rows + R - 1) / R);
        p.per_copy = p.grid;
        p.lds = 3072 + (uint32_t)((cols + 255) / 256 * 1024);
        return p;
    }
    // lanes a row: enough to cover a row's units (64-element chunks, or
    // 32-element blocks for Q8_0) in one sweep where the row allows
    const int64_t units = (type == CJ_Q4_K || type == CJ_Q6_K) ? cols / 256 * 4 : cols / 32;
    const int lpr = units >= 64 ? 64 : units >= 32 ? 32 : units >= 16 ? 16 : 8;
    const int groups = 64 / lpr;
    // rows in flight per lane group: 4, or 2 where the target asks for fewer
    // rows a workgroup than a 4-row pass covers (more workgroups on short
    // matrices); Q6_K always 2 (register budget)
    const int nr = type == CJ_Q6_K || target < 4 * groups * 4 ? 2 : 4;
    const int pass = 4 * groups * nr;                  // rows one pass of the workgroup covers
    int R = target > pass ? target / pass * pass : pass;
    while (R > 256) R -= pass;                         // one phase-B thread a row
    if (R < pass) R = pass;
    p.rows_per_wg = R;
    // a Q6_K row wider than one sweep: the form that requests the next
    // sweep's weights before the current sweep's arithmetic (4096×14336:
    // 27.9 → 20.4 µs; for Q8_0 it measured even to 5% slower)
    p.kernel = std::string(fam) + "_l" + std::to_string(lpr) + (nr == 2 && type != CJ_Q6_K ? "_n2" : "") +
               (type == CJ_Q6_K && lpr == 64 && units > 64 ? "_s" : "");
    p.grid = (uint32_t)((rows + R - 1) / R);
    p.per_copy = p.grid;
    // LDS: scratch, the staged pack, then R rows of block terms
    const int64_t terms = type == CJ_Q4_K ? cols / 256 * 2 : type == CJ_Q6_K ? cols / 256 : (cols / 32 + 7) / 8;
    p.lds = 3072 + (uint32_t)((cols + 255) / 256 * 320) + (uint32_t)(R * terms * 4);
    return p;
}

bool gemm_supported(int type) { return type == CJ_Q8_0 || type == CJ_Q4_K || type == CJ_Q6_K; }

// Two kernels, chosen by shape. The tiled kernel (4 waves a 64-row ×
// 16·NT-column tile over LDS-staged packs) when the row blocks and column
// tiles make at least 256 workgroups (a CU's worth each) — tall projections,
// many columns; otherwise the split-K kernel (8 waves sharing a 16-row
// tile's K dimension), which makes 4× more, smaller workgroups for short,
// wide products at few columns. Measured on MI355X at 32 columns (Q8_0):
// gate|up and head 2.1-2.3 TB/s tiled vs 1.1 split-K; q|k|v, o and down
// 0.8-1.1 TB/s split-K vs 0.3-0.5 tiled.
int run_gemm(const cj_gemv_args &a) {
    if (!gemm_supported(a.type) && a.type != CJ_Q4_0) return fail(CJ_ERR_ARG, "gemm: type %d is not served", a.type);
    if (a.batch <= 0 || a.rows <= 0) return fail(CJ_ERR_ARG, "gemm: %d columns, %lld rows", a.batch, (long long)a.rows);
    char name[32];
    if (a.type == CJ_Q4_0) {
        // many-column GEMV over f32 columns: 4·RW rows a workgroup, 4 columns a
        // grid row; RW = 4, or 2 where 4 would leave under two workgroups a CU
        // (measured at 4096x4096: 4 columns 11.3 -> 10.7 us; 16 columns 4 rows a wave 24.4 us, 2: 28.6)
        if (a.cols % 32) return fail(CJ_ERR_ARG, "gemm: Q4_0 rows are whole 32-element blocks");
        const int64_t cgroups = (a.batch + 3) / 4;
        if (cgroups > 65535) return fail(CJ_ERR_ARG, "gemm: %d columns exceed the grid", a.batch);
        const int rw = (a.rows + 15) / 16 * cgroups >= 2 * (int64_t)std::max(1, g.cus) ? 4 : 2;
        snprintf(name, sizeof name, "cj_gemm_q40_r%d_c4", rw);
        return launch2(name, (uint32_t)((a.rows + 4 * rw - 1) / (4 * rw)), (uint32_t)cgroups, 256, 0, a);
    }
    if (a.type == CJ_Q6_K) {
        // many-column GEMV (4 or 8 columns a grid row; its LDS fixed: a
        // 16-block sweep of the columns and the waves' terms), or above 8
        // columns the matrix-core form, 16 a grid row; 16 rows a workgroup
        const int nc = a.batch <= 4 ? 4 : a.batch <= 8 ? 8 : 16;
        if (a.cols % 256) return fail(CJ_ERR_ARG, "gemm: Q6_K rows are whole 256-element blocks");
        if ((a.batch + nc - 1) / nc > 65535) return fail(CJ_ERR_ARG, "gemm: %d columns exceed the grid", a.batch);
        if (nc == 16) snprintf(name, sizeof name, "cj_gemm_q6k_m16");
        else snprintf(name, sizeof name, "cj_gemm_q6k_c%d", nc);
        return launch2(name, (uint32_t)((a.rows + 15) / 16), (uint32_t)((a.batch + nc - 1) / nc), 256, 0, a);
    }
    const char *fmt = a.type == CJ_Q8_0 ? "q80" : "q4k";
    // Q4_K's 64-column tile needs more registers than two waves a SIMD leave
    const int nt = (a.batch <= 32 || a.type == CJ_Q4_K) ? 2 : 4;
    const int64_t tiles = ((a.rows + 63) / 64) * ((a.batch + 16 * nt - 1) / (16 * nt));
    if (tiles < 256 && a.batch <= 64) {
        const int sn = (a.type == CJ_Q8_0 && a.batch > 16) ? 2 : 1;
        const uint32_t gx = (uint32_t)((a.batch + 16 * sn - 1) / (16 * sn)), gy = (uint32_t)((a.rows + 15) / 16);
        if (gy > 65535) return fail(CJ_ERR_ARG, "gemm: %lld rows exceed the grid", (long long)a.rows);
        snprintf(name, sizeof name, "cj_gemm_sk_%s_n%d", fmt, sn);
        return launch2(name, gx, gy, 512, 0, a);
    }
    const uint32_t gx = (uint32_t)((a.batch + 16 * nt - 1) / (16 * nt)), gy = (uint32_t)((a.rows + 63) / 64);
    if (gy > 65535) return fail(CJ_ERR_ARG, "gemm: %lld rows exceed the grid", (long long)a.rows);
    snprintf(name, sizeof name, "cj_gemm_%s_n%d", fmt, nt);
    return launch2(name, gx, gy, 256, 0, a);
}

int run_gemv(const cj_gemv_args &a0, const GemvPlan &p) {
    cj_gemv_args a = a0;
    a.rows_per_wg = p.rows_per_wg;
    if (p.lds > 65536) return fail(CJ_ERR_ARG, "gemv %s: %u bytes of LDS exceed 64 KB", p.kernel.c_str(), p.lds);
    if (is_f32_act(a.type) && a.cols % 32)
        return fail(CJ_ERR_ARG, "gemv %s: %lld columns are not whole 32-element blocks", p.kernel.c_str(), (long long)a.cols);
    const uint32_t grid = (a.sel || a.route_logits) ? p.per_copy * (uint32_t)a.n_sel : p.grid;
    return launch(p.kernel.c_str(), grid, 256, p.lds, a);
}

}  // namespace cj

using namespace cj;

// ======================================================================= C-ABI

extern "C" {

int32_t cj_init(int32_t device) {
    if (ready()) return g.device == device ? CJ_OK : fail(CJ_ERR_STATE, "already initialised on device %d", g.device);
    CJ_HIP(hipSetDevice(device));
    hipDeviceProp_t pr;
    CJ_HIP(hipGetDeviceProperties(&pr, device));
    g.cus = pr.multiProcessorCount;
    g.hbm = (int64_t)pr.totalGlobalMem;
    g.lds = (int64_t)pr.maxSharedMemoryPerMultiProcessor;
    std::string path = module_path();
    hipError_t e = hipModuleLoad(&g.module, path.c_str());
    if (e != hipSuccess) {
        g.module = nullptr;
        return fail(CJ_ERR_NOKERNEL, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
    }
    static const char *kernels[] = {

        "cj_gemv_q6k_l64", "cj_gemv_q6k_l32", "cj_gemv_q6k_l16", "cj_gemv_q6k_l8",
        "cj_gemv_q80_l64", "cj_gemv_q80_l32", "cj_gemv_q80_l16", "cj_gemv_q80_l8",
        "cj_gemv_q80_l64_n2", "cj_gemv_q80_l32_n2", "cj_gemv_q80_l16_n2", "cj_gemv_q80_l8_n2",
        "cj_gemv_q6k_l64_s",
        "cj_gemv_q40b_r2", "cj_gemv_q40b_r4", "cj_gemm_q40_r2_c4", "cj_gemm_q40_r4_c4",
        "cj_gemv_mxfp4", "cj_gemv_f32", "cj_gemv_mxfp4_r32", "cj_gemv_f32_r32", "cj_gemv_mxfp4_r1", "cj_gemv_f32_r1",
        "cj_moe_combine", "cj_moe_combine_norm",
        "cj_pack", "cj_norm_pack", "cj_norm_pack_rows", "cj_copy", "cj_glu", "cj_add", "cj_dequant", "cj_prepare", "cj_embed", "cj_argmax",
        "cj_attn_split_h128_g4", "cj_attn_split_h128_g8", "cj_attn_scores_h64", "cj_attn_scores_h128",
        "cj_attn_combine_h64", "cj_attn_combine_h128", "cj_attn_fused_h64", "cj_attn_fused_h128",
        "cj_attn_merge", "cj_attn_merge_q", "cj_moe_group", "cj_argmax_pick", "cj_qkprep", "cj_zero", "cj_moe_route", "cj_router_topk",
        "cj_gemm_q80_n2", "cj_gemm_q4k_n2", "cj_gemm_q80_n4", "cj_gemm_q6k_c4", "cj_gemm_q6k_c8", "cj_gemm_q6k_m16",
        "cj_gemm_sk_q80_n1", "cj_gemm_sk_q80_n2", "cj_gemm_sk_q4k_n1",
        "cj_rows_embed", "cj_rows_qkv", "cj_rows_glu", "cj_rows_argmax", "cj_rows_pick",
        "cj_attn_split_rows_h128_g4", "cj_attn_split_rows_h128_g8", "cj_attn_merge_rows",
        "cj_attn_prefill_h128_g1", "cj_attn_prefill_h128_g2", "cj_attn_prefill_h128_g4", "cj_attn_prefill_h128_g8",
        "cj_attn_scores_rows_h64", "cj_attn_scores_rows_h128", "cj_attn_combine_rows_h64", "cj_attn_combine_rows_h128",
        "cj_attn_fused_rows_h64", "cj_attn_fused_rows_h128", "cj_attn_combine_grp_rows_h64", "cj_attn_combine_grp_rows_h128",
        "cj_attn_scores_grp_rows_h64", "cj_attn_scores_grp_rows_h128",
        "cj_attn_scores_f32_h64", "cj_attn_scores_f32_h128", "cj_attn_combine_f32_h64", "cj_attn_combine_f32_h128",
        "cj_attn_scores_rows_f32_h64", "cj_attn_scores_rows_f32_h128", "cj_attn_combine_rows_f32_h64",
        "cj_attn_combine_rows_f32_h128",
    };
    for (const char *k : kernels) {
        hipFunction_t f;
        if (hipModuleGetFunction(&f, g.module, k) == hipSuccess) g.fns[k] = f;
    }
    // MXFP4 experts grouped by expert: epilogue {g, s} × blocks a lane a sweep
    for (const char *e : {"g", "s"})
        for (const char *kb : {"1", "2", "3", "4"})
            for (const char *rt : {"32", "64", "128"}) {
                const std::string k = std::string("cj_moe_mxq8_") + e + "_k" + kb + "_t" + rt;
                hipFunction_t f;
                if (hipModuleGetFunction(&f, g.module, k.c_str()) == hipSuccess) g.fns[k] = f;
            }
    for (const char *k : {"cj_moe_mxq8_g_k3_t64_r1_c4", "cj_moe_mxq8_g_k3_t64_r2_c4", "cj_moe_mxq8_s_k3_t32_r1_c4",
                          "cj_moe_mxq8_s_k3_t32_r2_c4"}) {
        hipFunction_t f;
        if (hipModuleGetFunction(&f, g.module, k) == hipSuccess) g.fns[k] = f;
    }
    // MXFP4 × q8: epilogue {s, a, g} × blocks a lane a sweep
    for (const char *e : {"s", "a", "g"})
        for (const char *kb : {"1", "2", "3", "4"})
            for (const char *rw : {"2", "4"}) {
                const std::string k = std::string("cj_gemv_mxq8_") + e + "_k" + kb + "_r" + rw;
                hipFunction_t f;
                if (hipModuleGetFunction(&f, g.module, k.c_str()) == hipSuccess) g.fns[k] = f;
            }
    // the Q4_K family: prologue {c, p, n} × epilogue {s, a, q, g, m} × width
    for (const char *pro : {"c", "p", "n"})
        for (const char *epi : {"s", "a", "q", "g", "m"})
            for (const char *w : {"_b16", "_b8", "_b16_w", "_b64_w"})
                for (const char *it : {"", "_i1", "_i2", "_i4", "_i7"}) {
                    const std::string k = std::string("cj_gemv_q4k_") + pro + epi + w + it;
                    hipFunction_t f;
                    if (hipModuleGetFunction(&f, g.module, k.c_str()) == hipSuccess) g.fns[k] = f;
                }
    CJ_HIP(hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking));
    g.device = device;
    void *sp = nullptr;
    int rc = scratch_here(&sp);   // the allocation-free entry point's scratch, set up with the device current
    if (rc) return rc;
    return CJ_OK;
}

int32_t cj_shutdown(void) {
    if (!ready()) return CJ_OK;
    (void)hipStreamSynchronize(g.stream);
    std::vector<uintptr_t> ps;
    {
        std::lock_guard<std::mutex> lk(g.mu);
        for (auto &kv : g.allocs) ps.push_back(kv.first);
        g.allocs.clear();
    }
    for (auto p : ps) (void)hipFree((void *)p);
    (void)hipStreamDestroy(g.stream);
    (void)hipModuleUnload(g.module);
    g.module = nullptr;
    g.fns.clear();
    g.device = -1;
    return CJ_OK;
}

int32_t cj_last_error(int8_t *buf, int32_t cap) {
    if (!buf || cap <= 0) return CJ_ERR_ARG;
    snprintf((char *)buf, (size_t)cap, "%s", g_err.c_str());
    return CJ_OK;
}

int32_t cj_kernel_available(const int8_t *name) {
    if (!name || !ready()) return 0;
    std::string n((const char *)name);
    auto it = name_map().find(n);
    if (it != name_map().end()) n = it->second;
    return g.fns.count(n) ? 1 : 0;
}

int32_t cj_device_info(int64_t *out, int32_t n) {
    if (!ready()) return fail(CJ_ERR_STATE, "cj_init has not run");
    int64_t v[3] = {g.cus, g.hbm, g.lds};
    for (int i = 0; i < n && i < 3; i++) out[i] = v[i];
    return CJ_OK;
}

// ------------------------------------------------------------- buffers

int64_t cj_buf_alloc(int64_t bytes) {
    if (!ready()) return fail(CJ_ERR_STATE, "cj_init has not run"), 0;
    if (bytes <= 0) return fail(CJ_ERR_ARG, "cj_buf_alloc: %lld bytes", (long long)bytes), 0;
    void *p = dev_alloc((size_t)bytes);
    if (!p) return fail(CJ_ERR_HIP, "hipMalloc(%lld) failed", (long long)bytes), 0;
    return (int64_t)(uintptr_t)p;
}

int32_t cj_buf_free(int64_t buf) {
    std::lock_guard<std::mutex> lk(g.mu);
    auto it = g.allocs.find((uintptr_t)buf);
    if (it == g.allocs.end()) return fail(CJ_ERR_STATE, "cj_buf_free: unknown handle");
    g.allocs.erase(it);
    (void)hipFree((void *)(uintptr_t)buf);
    return CJ_OK;
}

int64_t cj_buf_size(int64_t buf) {
    std::lock_guard<std::mutex> lk(g.mu);
    auto it = g.allocs.find((uintptr_t)buf);
    return it == g.allocs.end() ? 0 : (int64_t)it->second;
}

int32_t cj_buf_upload(int64_t buf, int64_t off, const int8_t *src, int64_t bytes) {
    if (!in_buffer(dptr(buf + off), bytes)) return fail(CJ_ERR_ARG, "cj_buf_upload: extent outside the buffer");
    CJ_HIP(hipMemcpyAsync(dptr(buf + off), src, (size_t)bytes, hipMemcpyHostToDevice, g.stream));
    CJ_HIP(hipStreamSynchronize(g.stream));
    return CJ_OK;
}

int32_t cj_buf_download(int64_t buf, int64_t off, int8_t *dst, int64_t bytes) {
    if (!in_buffer(dptr(buf + off), bytes)) return fail(CJ_ERR_ARG, "cj_buf_download: extent outside the buffer");
    CJ_HIP(hipMemcpyAsync(dst, dptr(buf + off), (size_t)bytes, hipMemcpyDeviceToHost, g.stream));
    CJ_HIP(hipStreamSynchronize(g.stream));
    return CJ_OK;
}

int32_t cj_buf_zero(int64_t buf) {
    int64_t n = cj_buf_size(buf);
    if (n <= 0) return fail(CJ_ERR_ARG, "cj_buf_zero: unknown handle");
    struct { uint32_t *p; int64_t words; } a = {(uint32_t *)dptr(buf), (n + 3) / 4};
    uint32_t grid = (uint32_t)std::min<int64_t>((a.words + 255) / 256, 65535);
    return launch("cj_zero", grid, 256, 0, a);
}

// -------------------------------------------------------- stream / graph

int32_t cj_stream_sync(void) {
    if (!ready()) return fail(CJ_ERR_STATE, "cj_init has not run");
    CJ_HIP(hipStreamSynchronize(g.stream));
    return CJ_OK;
}

int32_t cj_graph_begin(void) {
    if (!ready()) return fail(CJ_ERR_STATE, "cj_init has not run");
    CJ_HIP(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal));
    return CJ_OK;
}

int64_t cj_graph_end(void) {
    hipGraph_t gr = nullptr;
    hipError_t e = hipStreamEndCapture(g.stream, &gr);
    if (e != hipSuccess) return fail(CJ_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e)), 0;
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0);
    (void)hipGraphDestroy(gr);
    if (e != hipSuccess) return fail(CJ_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e)), 0;
    return (int64_t)(uintptr_t)ex;
}

int32_t cj_graph_launch(int64_t graph) {
    if (!graph) return fail(CJ_ERR_ARG, "cj_graph_launch: null graph");
    CJ_HIP(hipGraphLaunch((hipGraphExec_t)(uintptr_t)graph, g.stream));
    return CJ_OK;
}

int32_t cj_graph_free(int64_t graph) {
    if (graph) CJ_HIP(hipGraphExecDestroy((hipGraphExec_t)(uintptr_t)graph));
    return CJ_OK;
}

int64_t cj_event_record(void) {
    hipEvent_t ev;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) return fail(CJ_ERR_HIP, "hipEventCreate"), 0;
    if (hipEventRecord(ev, g.stream) != hipSuccess) return fail(CJ_ERR_HIP, "hipEventRecord"), 0;
    return (int64_t)(uintptr_t)ev;
}
int32_t cj_event_wait(int64_t ev) {
    CJ_HIP(hipEventSynchronize((hipEvent_t)(uintptr_t)ev));
    return CJ_OK;
}
int32_t cj_event_free(int64_t ev) {
    CJ_HIP(hipEventDestroy((hipEvent_t)(uintptr_t)ev));
    return CJ_OK;
}

// --------------------------------------------------------- launch seam

int32_t cj_q8k_pack(int64_t out, int64_t x, int64_t rows, int64_t n, int64_t npad, int32_t per32) {
    if (rows <= 0 || n <= 0 || npad < n || npad % 256) return fail(CJ_ERR_ARG, "cj_q8k_pack: rows %lld n %lld npad %lld", (long long)rows, (long long)n, (long long)npad);
    if (npad / 256 > 64) return fail(CJ_ERR_ARG, "cj_q8k_pack: %lld columns exceed the 16384 staged", (long long)npad);
    if (!in_buffer(dptr(x), rows * n * 4) || !in_buffer(dptr(out), rows * npad / 256 * 320))
        return fail(CJ_ERR_ARG, "cj_q8k_pack: buffers smaller than %lld rows", (long long)rows);
    cj_pack_args a{};
    a.out = (uint8_t *)dptr(out); a.x = (const float *)dptr(x); a.n = n; a.npad = npad; a.rows = rows; a.per32 = per32;
    return launch("cj_pack", (uint32_t)rows, 256, (uint32_t)(npad / 256 * 320), a);
}

int32_t cj_rmsnorm_pack(int64_t out, int64_t packed, int64_t x, int64_t w, int64_t dim, float eps, int32_t form, int32_t per32) {
    if (dim <= 0 || (!out && !packed)) return fail(CJ_ERR_ARG, "cj_rmsnorm_pack: dim %lld", (long long)dim);
    const int64_t npad = (dim + 255) / 256 * 256;
    if (npad / 256 > 64) return fail(CJ_ERR_ARG, "cj_rmsnorm_pack: %lld columns exceed the 16384 staged", (long long)dim);
    if (!in_buffer(dptr(x), dim * 4) || !in_buffer(dptr(w), dim * 4) || (out && !in_buffer(dptr(out), dim * 4)) ||
        (packed && !in_buffer(dptr(packed), npad / 256 * 320)))
        return fail(CJ_ERR_ARG, "cj_rmsnorm_pack: a buffer is smaller than dim %lld needs", (long long)dim);
    cj_pack_args a{};
    a.out = (uint8_t *)dptr(packed); a.x = (const float *)dptr(x); a.w = (const float *)dptr(w);
    a.xout = (float *)dptr(out); a.n = dim; a.npad = npad; a.rows = 1; a.eps = eps; a.form = form; a.per32 = per32; a.do_norm = 1;
    return launch("cj_pack", 1, 256, (uint32_t)(npad / 256 * 320), a);
}

int64_t cj_prepared_row_bytes(int32_t type, int64_t cols) { return prepared_row_bytes(type, cols); }

int32_t cj_prepare_weight(int64_t dst, int64_t src, int32_t type, int64_t rows, int64_t cols) {
    const int64_t prb = prepared_row_bytes(type, cols);
    if (prb <= 0 || rows <= 0) return fail(CJ_ERR_ARG, "cj_prepare_weight: type %d cols %lld", type, (long long)cols);
    const int64_t be = (type == CJ_Q4_K || type == CJ_Q6_K) ? 256 : 32;
    const int64_t bb = type == CJ_Q4_K ? 144 : type == CJ_Q6_K ? 210 : type == CJ_Q8_0 ? 34 : type == CJ_Q4_0 ? 18 : 17;
    const int64_t srb = cols / be * bb;
    if (!in_buffer(dptr(src), rows * srb) || !in_buffer(dptr(dst), rows * prb))
        return fail(CJ_ERR_ARG, "cj_prepare_weight: buffers smaller than %lld rows", (long long)rows);
    cj_prepare_args a{};
    a.dst = (uint8_t *)dptr(dst); a.src = (const uint8_t *)dptr(src); a.rows = rows; a.cols = cols;
    a.src_row_bytes = srb; a.dst_row_bytes = prb; a.type = type;
    const int64_t items = rows * (cols / be);
    return launch("cj_prepare", (uint32_t)((items + 255) / 256), 256, 0, a);
}

int32_t cj_matvec(int32_t type, int64_t y, int64_t w, int64_t act, int64_t rows, int64_t cols, int64_t y_off, int32_t accum) {
    const int64_t prb = prepared_row_bytes(type, cols);
    if (prb <= 0 || rows <= 0 || !gemv_supported(type, cols))
        return fail(CJ_ERR_ARG, "cj_matvec: type %d with %lld columns is not served", type, (long long)cols);
    const int64_t nblk = (cols + 255) / 256;
    const bool f32 = is_f32_act(type);
    if (!in_buffer(dptr(w), rows * prb)) return fail(CJ_ERR_ARG, "cj_matvec: weight smaller than %lld prepared rows", (long long)rows);
    if (!in_buffer(dptr(act), f32 ? cols * 4 : nblk * 320)) return fail(CJ_ERR_ARG, "cj_matvec: activation smaller than its %s form", f32 ? "f32" : "packed");
    if (y_off < 0 || !in_buffer(dptr(y + 4 * y_off), rows * 4)) return fail(CJ_ERR_ARG, "cj_matvec: output smaller than y_off + rows");
    cj_gemv_args a{};
    a.w = (const uint8_t *)dptr(w);
    if (f32) { a.x = (const float *)dptr(act); a.pro = CJ_PRO_F32; }
    else { a.xp = (const uint8_t *)dptr(act); a.pro = CJ_PRO_PACKED; }
    a.y = (float *)dptr(y); a.y_off = y_off; a.rows = rows; a.cols = cols; a.row_bytes = prb; a.type = type;
    a.epi = accum ? CJ_EPI_ACCUM : CJ_EPI_STORE; a.per32 = type == CJ_Q8_0; a.batch = 1;
    return run_gemv(a, plan_gemv(type, rows, cols, 32, a.pro, a.epi));
}

int32_t cj_matvec_mxfp4_q8(int64_t y, int64_t w, int64_t x, int64_t rows, int64_t cols, int64_t y_off, int32_t accum) {
    const int64_t prb = prepared_row_bytes(CJ_MXFP4, cols);
    if (prb <= 0 || rows <= 0) return fail(CJ_ERR_ARG, "cj_matvec_mxfp4_q8: %lld columns are not whole 32-element blocks", (long long)cols);
    if (!in_buffer(dptr(w), rows * prb)) return fail(CJ_ERR_ARG, "cj_matvec_mxfp4_q8: weight smaller than %lld prepared rows", (long long)rows);
    if (!in_buffer(dptr(x), cols * 4) || ((uintptr_t)dptr(x) & 15))
        return fail(CJ_ERR_ARG, "cj_matvec_mxfp4_q8: activation smaller than %lld floats or not 16-byte aligned", (long long)cols);
    if (y_off < 0 || !in_buffer(dptr(y + 4 * y_off), rows * 4)) return fail(CJ_ERR_ARG, "cj_matvec_mxfp4_q8: output smaller than y_off + rows");
    cj_gemv_args a{};
    a.w = (const uint8_t *)dptr(w); a.x = (const float *)dptr(x); a.y = (float *)dptr(y); a.y_off = y_off;
    a.rows = rows; a.cols = cols; a.row_bytes = prb; a.type = CJ_MXFP4; a.pro = CJ_PRO_MXQ8;
    a.epi = accum ? CJ_EPI_ACCUM : CJ_EPI_STORE; a.batch = 1;
    return run_gemv(a, plan_gemv(CJ_MXFP4, rows, cols, 32, a.pro, a.epi));
}

int32_t cj_matmul(int32_t type, int64_t y, int64_t w, int64_t xp, int64_t rows, int64_t cols, int32_t ncols,
                  int64_t xp_stride, int64_t y_stride, int64_t y_off, int32_t accum) {
    const int64_t prb = prepared_row_bytes(type, cols);
    const bool f32cols = type == CJ_Q4_0;      // f32 activation columns (the format reads f32)
    if (!(gemm_supported(type) || f32cols) || prb <= 0 || rows <= 0 || ncols <= 0)
        return fail(CJ_ERR_ARG, "cj_matmul: type %d with %lld columns x %d is not served", type, (long long)cols, ncols);
    const int64_t pack_bytes = f32cols ? cols * 4 : (cols + 255) / 256 * 320;
    if (xp_stride < pack_bytes || y_stride < y_off + rows || y_off < 0)
        return fail(CJ_ERR_ARG, "cj_matmul: strides %lld/%lld smaller than one column", (long long)xp_stride, (long long)y_stride);
    if (!in_buffer(dptr(w), rows * prb)) return fail(CJ_ERR_ARG, "cj_matmul: weight smaller than %lld prepared rows", (long long)rows);
    if (!in_buffer(dptr(xp), (ncols - 1) * xp_stride + pack_bytes)) return fail(CJ_ERR_ARG, "cj_matmul: activation packs too small");
    if (!in_buffer(dptr(y), ((ncols - 1) * y_stride + y_off + rows) * 4)) return fail(CJ_ERR_ARG, "cj_matmul: output too small");
    cj_gemv_args a{};
    a.w = (const uint8_t *)dptr(w); a.xp = (const uint8_t *)dptr(xp); a.y = (float *)dptr(y);
    a.rows = rows; a.cols = cols; a.row_bytes = prb; a.type = type; a.batch = ncols;
    a.xp_stride = xp_stride; a.y_stride = y_stride; a.y_off = y_off;
    a.epi = accum ? CJ_EPI_ACCUM : CJ_EPI_STORE; a.pro = f32cols ? CJ_PRO_F32 : CJ_PRO_PACKED;
    return run_gemm(a);
}

int32_t cj_glu(int64_t out, int64_t packed, int64_t gb, int64_t ub, int64_t n, int32_t form, int32_t per32) {
    const int64_t npad = (n + 255) / 256 * 256;
    if (n <= 0 || !in_buffer(dptr(out), n * 4) || !in_buffer(dptr(gb), n * 4) || !in_buffer(dptr(ub), n * 4) ||
        (packed && !in_buffer(dptr(packed), npad / 256 * 320)))
        return fail(CJ_ERR_ARG, "cj_glu: buffers smaller than n %lld", (long long)n);
    cj_glu_args a{};
    a.out = (float *)dptr(out); a.g = (const float *)dptr(gb); a.u = (const float *)dptr(ub);
    a.packed = (uint8_t *)dptr(packed); a.n = n; a.npad = npad; a.form = form; a.per32 = per32;
    return launch("cj_glu", (uint32_t)(npad / 256), 256, 0, a);
}

int32_t cj_buf_copy(int64_t dst, int64_t src, int64_t bytes) {
    if (bytes <= 0 || bytes % 16 || (dst & 15) || (src & 15) || !in_buffer(dptr(dst), bytes) || !in_buffer(dptr(src), bytes))
        return fail(CJ_ERR_ARG, "cj_buf_copy: %lld bytes (a multiple of 16, 16-byte aligned, inside both buffers)",
                    (long long)bytes);
    cj_copy_args a{dptr(dst), dptr(src), bytes / 16};
    const int64_t wgs = std::min<int64_t>((a.n16 + 255) / 256, (int64_t)std::max(1, g.cus) * 16);
    return launch("cj_copy", (uint32_t)wgs, 256, 0, a);
}

int32_t cj_add(int64_t ab, int64_t bb, int64_t n) {
    if (n <= 0 || !in_buffer(dptr(ab), n * 4) || !in_buffer(dptr(bb), n * 4)) return fail(CJ_ERR_ARG, "cj_add: n %lld", (long long)n);
    cj_add_args a{(float *)dptr(ab), (const float *)dptr(bb), n};
    return launch("cj_add", (uint32_t)((n + 255) / 256), 256, 0, a);
}

int32_t cj_rope_table(int64_t out, int32_t head_dim, float theta, int32_t ctx) {
    return cj_rope_table_freqs(out, head_dim, theta, ctx, nullptr, 0);
}

int32_t cj_rope_table_freqs(int64_t out, int32_t head_dim, float theta, int32_t ctx, const float *freqs, int32_t n_freqs) {
    const int half = head_dim / 2;
    if (head_dim <= 0 || head_dim % 2 || ctx <= 0 || !in_buffer(dptr(out), (int64_t)ctx * half * 8))
        return fail(CJ_ERR_ARG, "cj_rope_table: head_dim %d ctx %d", head_dim, ctx);
    if (freqs && n_freqs != half)
        return fail(CJ_ERR_ARG, "rope_freqs has %d entries; expected %d (headDim/2)", n_freqs, half);
    std::vector<float> inv(half), tab((size_t)ctx * half * 2);
    for (int d = 0; d < half; d++) inv[d] = powf(theta, (0.0f - (float)(2 * d)) / (float)head_dim);
    // precomputed per-dimension factors: theta_d /= factor_d (a zero factor
    // leaves the dimension as it is)
    if (freqs)
        for (int d = 0; d < half; d++)
            if (freqs[d] != 0.0f) inv[d] = inv[d] / freqs[d];
    for (int p = 0; p < ctx; p++)
        for (int d = 0; d < half; d++) {
            const float ang = (float)p * inv[d];
            tab[((size_t)p * half + d) * 2] = cosf(ang);
            tab[((size_t)p * half + d) * 2 + 1] = sinf(ang);
        }
    return cj_buf_upload(out, 0, (const int8_t *)tab.data(), (int64_t)tab.size() * 4);
}

int32_t cj_qk_prep(int64_t q, int64_t k, int64_t v, int64_t kcache, int64_t vcache, int64_t qw, int64_t kw,
                   int64_t rope, int64_t pgtab, int32_t pg_base, int32_t n_q, int32_t n_kv, int32_t head_dim,
                   int32_t norm, float eps, int32_t form, int32_t pos) {
    if (n_q <= 0 || n_kv <= 0 || head_dim <= 0 || head_dim % 2 || head_dim > 256 || pos < 0)
        return fail(CJ_ERR_ARG, "cj_qk_prep: heads %d/%d hd %d pos %d", n_q, n_kv, head_dim, pos);
    const int64_t page = pos / 64;
    if (!in_buffer(dptr(q), (int64_t)n_q * head_dim * 4) || !in_buffer(dptr(k), (int64_t)n_kv * head_dim * 4) ||
        !in_buffer(dptr(v), (int64_t)n_kv * head_dim * 4) || !in_buffer(dptr(pgtab + 4 * (pg_base + page)), 4) ||
        !in_buffer(dptr(rope), ((int64_t)pos + 1) * head_dim * 4) ||
        (norm && (!in_buffer(dptr(qw), head_dim * 4) || !in_buffer(dptr(kw), head_dim * 4))))
        return fail(CJ_ERR_ARG, "cj_qk_prep: a buffer is smaller than the shapes need");
    int32_t pg = 0;
    CJ_HIP(hipMemcpyAsync(&pg, dptr(pgtab + 4 * (pg_base + page)), 4, hipMemcpyDeviceToHost, g.stream));
    CJ_HIP(hipStreamSynchronize(g.stream));
    const int64_t need = (((int64_t)pg + 1) * n_kv * 64) * head_dim * 2;
    if (pg < 0 || !in_buffer(dptr(kcache), need) || !in_buffer(dptr(vcache), need))
        return fail(CJ_ERR_CAPACITY, "cj_qk_prep: page %d outside the K/V planes", pg);
    cj_qkprep_args a{};
    a.q = (float *)dptr(q); a.k = (float *)dptr(k); a.v = (const float *)dptr(v);
    a.kc = (uint16_t *)dptr(kcache); a.vc = (uint16_t *)dptr(vcache); a.qw = (const float *)dptr(qw); a.kw = (const float *)dptr(kw);
    a.rope_cs = (const float *)dptr(rope); a.pgtab = (const int32_t *)dptr(pgtab);
    a.n_q = n_q; a.n_kv = n_kv; a.head_dim = head_dim; a.norm = norm; a.form = form; a.pg_base = pg_base; a.pos = pos; a.eps = eps;
    return launch("cj_qkprep", (uint32_t)(n_q + n_kv), 64, 0, a);
}

int32_t cj_attend(int64_t part, int64_t out, int64_t q, int64_t kcache, int64_t vcache, int64_t pgtab, int32_t pg_base,
                  int64_t counters, int32_t n_q, int32_t n_kv, int32_t head_dim, int32_t count, int32_t from,
                  int32_t workers, float scale) {
    if (n_kv <= 0 || n_q <= 0 || n_q % n_kv || n_q / n_kv > 64 || (head_dim != 64 && head_dim != 128) || count <= 0 ||
        from < 0 || workers <= 0)
        return fail(CJ_ERR_ARG, "cj_attend: heads %d/%d hd %d count %d workers %d", n_q, n_kv, head_dim, count, workers);
    const int grp = n_q / n_kv;
    const bool split = head_dim == 128 && (grp == 4 || grp == 8);
    const int64_t pages = ((int64_t)from + count + 63) / 64;
    if (!split && (from + count - 1) / 64 - from / 64 + 1 > 2048)
        return fail(CJ_ERR_ARG, "cj_attend: %d positions from %d span more than 2048 pages", count, from);
    const int64_t part_bytes = split ? (int64_t)n_q * 64 * (head_dim + 2) * 4 : (int64_t)n_q * count * 4;
    if (!in_buffer(dptr(pgtab + 4 * pg_base), pages * 4) || !in_buffer(dptr(q), (int64_t)n_q * head_dim * 4) ||
        !in_buffer(dptr(part), part_bytes) || (!split && !out) ||
        (out && !in_buffer(dptr(out), (int64_t)n_q * head_dim * 4)) ||
        (split && out && !in_buffer(dptr(counters), (int64_t)n_kv * 4)))
        return fail(CJ_ERR_ARG, "cj_attend: a buffer is smaller than the shapes need");
    std::vector<int32_t> tab((size_t)pages);
    CJ_HIP(hipMemcpyAsync(tab.data(), dptr(pgtab + 4 * pg_base), (size_t)pages * 4, hipMemcpyDeviceToHost, g.stream));
    CJ_HIP(hipStreamSynchronize(g.stream));
    int32_t maxpg = 0;
    for (int32_t p : tab) {
        if (p < 0) return fail(CJ_ERR_ARG, "cj_attend: negative page in the table");
        maxpg = std::max(maxpg, p);
    }
    const int64_t need = (((int64_t)maxpg + 1) * n_kv * 64) * head_dim * 2;
    if (!in_buffer(dptr(kcache), need) || !in_buffer(dptr(vcache), need))
        return fail(CJ_ERR_ARG, "cj_attend: page %d outside the K/V planes", maxpg);
    cj_attn_args a{};
    a.part = (float *)dptr(part); a.out = (float *)dptr(out); a.q = (const float *)dptr(q);
    a.kc = (const uint16_t *)dptr(kcache); a.vc = (const uint16_t *)dptr(vcache); a.pgtab = (const int32_t *)dptr(pgtab);
    a.counters = (int32_t *)dptr(counters); a.n_q = n_q; a.n_kv = n_kv; a.head_dim = head_dim;
    a.pg_base = pg_base; a.pg_n = (int32_t)pages; a.count = count; a.from = from; a.window = 0; a.workers = workers; a.scale = scale;
    char name[64];
    if (split) {
        snprintf(name, sizeof name, "cj_attn_split_h128_g%d", grp);
        return launch(name, (uint32_t)(n_kv * 64), 256, 0, a);
    }
    a.splits = count;   // the scores row stride
    snprintf(name, sizeof name, "cj_attn_scores_h%d", head_dim);
    if (int32_t rc = launch2(name, (uint32_t)((count + 255) / 256), (uint32_t)n_q, 256, 0, a)) return rc;
    snprintf(name, sizeof name, "cj_attn_combine_h%d", head_dim);
    return launch(name, (uint32_t)(n_q * (head_dim / CJ_COMBINE_DH)), 256, 0, a);
}

int32_t cj_decode_splits(int32_t count, int32_t n_kv, int32_t workers) {
    const int w = workers < 1 ? 1 : workers, rk = n_kv < 1 ? 1 : n_kv;
    return std::max(1, std::min({64, count, (2 * w + rk - 1) / rk}));
}

int32_t cj_attn_merge(int64_t out, int64_t packed, int64_t part, int32_t n_q, int32_t head_dim, int32_t splits, int32_t per32) {
    const int64_t n = (int64_t)n_q * head_dim, npad = (n + 255) / 256 * 256;
    if (n <= 0 || head_dim % 64 || splits <= 0 || splits > 64 || !in_buffer(dptr(part), (int64_t)n_q * 64 * (head_dim + 2) * 4) ||
        (out && !in_buffer(dptr(out), n * 4)) || (packed && !in_buffer(dptr(packed), npad / 256 * 320)) || (!out && !packed))
        return fail(CJ_ERR_ARG, "cj_attn_merge: buffers smaller than the shapes need");
    cj_merge_args a{};
    a.out = (float *)dptr(out); a.packed = (uint8_t *)dptr(packed); a.part = (const float *)dptr(part);
    a.n_q = n_q; a.head_dim = head_dim; a.splits = splits; a.per32 = per32;
    return launch("cj_attn_merge", (uint32_t)(npad / 256), 256, 0, a);
}

int32_t cj_embed_row(int64_t out, int64_t table, int32_t type, int64_t hidden, int32_t token) {
    const int64_t be = (type == CJ_Q4_K || type == CJ_Q6_K) ? 256 : (type == CJ_F32 || type == CJ_F16) ? 1 : 32;
    const int64_t bb = type == CJ_F32 ? 4 : type == CJ_F16 ? 2 : type == CJ_Q4_K ? 144 : type == CJ_Q6_K ? 210
                     : type == CJ_Q8_0 ? 34 : type == CJ_Q4_0 ? 18 : type == CJ_MXFP4 ? 17 : -1;
    if (bb < 0 || hidden % be || token < 0) return fail(CJ_ERR_ARG, "cj_embed_row: type %d hidden %lld", type, (long long)hidden);
    const int64_t rb = hidden / be * bb;
    if (!in_buffer(dptr(table + ((int64_t)token) * rb), rb) || !in_buffer(dptr(out), hidden * 4))
        return fail(CJ_ERR_ARG, "cj_embed_row: token %d outside the table", token);
    cj_embed_args a{};
    a.out = (float *)dptr(out); a.table = (const uint8_t *)dptr(table); a.type = type; a.hidden = hidden; a.row_bytes = rb; a.token = token;
    return launch("cj_embed", (uint32_t)((hidden + 255) / 256), 256, 0, a);
}

int32_t cj_embed_row_slot(int64_t out, int64_t table, int32_t type, int64_t hidden, int32_t vocab, int64_t tokens,
                          int32_t slot, int64_t status) {
    const int64_t be = (type == CJ_Q4_K || type == CJ_Q6_K) ? 256 : (type == CJ_F32 || type == CJ_F16) ? 1 : 32;
    const int64_t bb = type == CJ_F32 ? 4 : type == CJ_F16 ? 2 : type == CJ_Q4_K ? 144 : type == CJ_Q6_K ? 210
                     : type == CJ_Q8_0 ? 34 : type == CJ_Q4_0 ? 18 : type == CJ_MXFP4 ? 17 : -1;
    if (bb < 0 || hidden <= 0 || hidden % be || vocab <= 0 || slot < 0)
        return fail(CJ_ERR_ARG, "cj_embed_row_slot: type %d hidden %lld vocab %d slot %d", type, (long long)hidden, vocab, slot);
    const int64_t rb = hidden / be * bb;
    if (!in_buffer(dptr(table), (int64_t)vocab * rb) || !in_buffer(dptr(out), hidden * 4) ||
        !in_buffer(dptr(tokens + 4 * (int64_t)slot), 4) || (status && !in_buffer(dptr(status), 4)))
        return fail(CJ_ERR_ARG, "cj_embed_row_slot: a buffer is smaller than its extent");
    cj_embed_args a{};
    a.out = (float *)dptr(out); a.table = (const uint8_t *)dptr(table); a.type = type; a.hidden = hidden; a.row_bytes = rb;
    a.tokens = (const int32_t *)dptr(tokens); a.state = nullptr; a.token = slot; a.vocab = vocab;
    a.status = status ? (int32_t *)dptr(status) : nullptr;
    return launch("cj_embed", (uint32_t)((hidden + 255) / 256), 256, 0, a);
}

int32_t cj_argmax_row(int64_t tok, int32_t row, int64_t v, int64_t n) {
    if (n <= 0 || row < 0 || !in_buffer(dptr(tok + 4 * row), 4) || !in_buffer(dptr(v), n * 4))
        return fail(CJ_ERR_ARG, "cj_argmax_row: n %lld row %d", (long long)n, row);
    // its scratch may grow (a synchronize, an allocation and a memset),
    // none of which a stream capture may record
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    CJ_HIP(hipStreamIsCapturing(g.stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(CJ_ERR_STATE, "cj_argmax_row: the stream is capturing a graph; cj_argmax_row_noalloc allocates nothing");
    static void *scratch = nullptr;
    static int64_t scratch_groups = 0;
    const int64_t groups = (n + 1023) / 1024;
    if (groups > scratch_groups) {
        CJ_HIP(hipStreamSynchronize(g.stream));
        dev_free(scratch);
        scratch = dev_alloc((size_t)(groups * 8 + 64));
        if (!scratch) return fail(CJ_ERR_HIP, "cj_argmax_row: scratch allocation");
        CJ_HIP(hipMemsetAsync(scratch, 0, (size_t)(groups * 8 + 64), g.stream));
        scratch_groups = groups;
    }
    cj_argmax_args a{};
    a.tok = (int32_t *)dptr(tok); a.v = (const float *)dptr(v); a.pv = (float *)scratch;
    a.pi = (int32_t *)((char *)scratch + scratch_groups * 4); a.counter = (int32_t *)((char *)scratch + scratch_groups * 8);
    a.n = n; a.row = row;
    return launch("cj_argmax", (uint32_t)groups, 256, 0, a);
}

int32_t cj_argmax_row_noalloc(int64_t tok, int32_t row, int64_t v, int64_t n) {
    if (!ready()) return fail(CJ_ERR_STATE, "cj_init has not run");
    if (n <= 0 || n > CJ_NOALLOC_ARGMAX_MAX)
        return fail(CJ_ERR_ARG, "cj_argmax_row_noalloc: n %lld outside 1..%d (the static scratch's limit)", (long long)n,
                    CJ_NOALLOC_ARGMAX_MAX);
    if (row < 0 || !in_buffer(dptr(tok + 4 * (int64_t)row), 4) || !in_buffer(dptr(v), n * 4))
        return fail(CJ_ERR_ARG, "cj_argmax_row_noalloc: n %lld row %d", (long long)n, row);
    void *sp = nullptr;
    int rc = scratch_here(&sp);
    if (rc) return rc;
    cj_argmax_args a{};
    a.tok = (int32_t *)dptr(tok); a.v = (const float *)dptr(v);
    a.pv = (float *)sp;
    a.pi = (int32_t *)((char *)sp + CJ_NOALLOC_GROUPS * 4);
    a.counter = (int32_t *)((char *)sp + CJ_NOALLOC_GROUPS * 8);
    a.n = n; a.row = row;
    return launch("cj_argmax", (uint32_t)((n + 1023) / 1024), 256, 0, a);
}

int32_t cj_dequant(int64_t out, int64_t raw, int32_t type, int64_t rows, int64_t cols, int32_t prepared) {
    int64_t rb;
    if (prepared) rb = prepared_row_bytes(type, cols);
    else {
        const int64_t be = (type == CJ_Q4_K || type == CJ_Q6_K) ? 256 : (type == CJ_F32 || type == CJ_F16) ? 1 : 32;
        const int64_t bb = type == CJ_F32 ? 4 : type == CJ_F16 ? 2 : type == CJ_Q4_K ? 144 : type == CJ_Q6_K ? 210
                         : type == CJ_Q8_0 ? 34 : type == CJ_Q4_0 ? 18 : type == CJ_MXFP4 ? 17 : -1;
        rb = (bb < 0 || cols % be) ? -1 : cols / be * bb;
    }
    if (rb <= 0 || rows <= 0) return fail(CJ_ERR_ARG, "cj_dequant: type %d cols %lld", type, (long long)cols);
    if (!in_buffer(dptr(raw), rows * rb) || !in_buffer(dptr(out), rows * cols * 4))
        return fail(CJ_ERR_ARG, "cj_dequant: buffers smaller than %lld rows", (long long)rows);
    cj_dequant_args a{};
    a.out = (float *)dptr(out); a.raw = (const uint8_t *)dptr(raw); a.elems = rows * cols; a.row_bytes = rb; a.cols = cols;
    a.type = type; a.prepared = prepared;
    const int64_t grid = std::min<int64_t>((a.elems + 255) / 256, 16384);
    return launch("cj_dequant", (uint32_t)grid, 256, 0, a);
}

int32_t cj_router_topk(int64_t sel, int64_t w, int64_t logits, int64_t w_router, int64_t x, int64_t counter,
                       int32_t experts, int32_t cols, int32_t used, int32_t norm_topk, float w_scale) {
    if (experts <= 0 || experts > 4096 || cols <= 0 || used <= 0 || used > experts ||
        !in_buffer(dptr(sel), (int64_t)used * 4) || !in_buffer(dptr(w), (int64_t)used * 4) ||
        !in_buffer(dptr(logits), (int64_t)experts * 4) || !in_buffer(dptr(w_router), (int64_t)experts * cols * 4) ||
        !in_buffer(dptr(x), (int64_t)cols * 4) || !in_buffer(dptr(counter), 4))
        return fail(CJ_ERR_ARG, "cj_router_topk: experts %d cols %d used %d", experts, cols, used);
    cj_router_topk_args a{};
    a.sel = (int32_t *)dptr(sel); a.w = (float *)dptr(w); a.logits = (float *)dptr(logits);
    a.w_router = (const float *)dptr(w_router); a.x = (const float *)dptr(x); a.counter = (int32_t *)dptr(counter);
    a.experts = experts; a.cols = cols; a.used = used; a.norm_topk = norm_topk ? 1 : 0; a.w_scale = w_scale;
    return launch("cj_router_topk", (uint32_t)experts, 256, 0, a);
}

int32_t cj_attn_scores(int64_t scores, int64_t q, int64_t kcache, int64_t pgtab, int32_t pg_base, int32_t n_q,
                       int32_t n_kv, int32_t head_dim, int32_t count, int32_t from, float scale) {
    if (n_kv <= 0 || n_q <= 0 || n_q % n_kv || (head_dim != 64 && head_dim != 128) || count <= 0 || from < 0)
        return fail(CJ_ERR_ARG, "cj_attn_scores: heads %d/%d hd %d count %d", n_q, n_kv, head_dim, count);
    const int64_t pages = ((int64_t)from + count + 63) / 64;
    if (!in_buffer(dptr(pgtab + 4 * (int64_t)pg_base), pages * 4) || !in_buffer(dptr(q), (int64_t)n_q * head_dim * 4) ||
        !in_buffer(dptr(scores), (int64_t)n_q * count * 4))
        return fail(CJ_ERR_ARG, "cj_attn_scores: a buffer is smaller than the shapes need");
    std::vector<int32_t> tab((size_t)pages);
    CJ_HIP(hipMemcpyAsync(tab.data(), dptr(pgtab + 4 * (int64_t)pg_base), (size_t)pages * 4, hipMemcpyDeviceToHost, g.stream));
    CJ_HIP(hipStreamSynchronize(g.stream));
    int32_t maxpg = 0;
    for (int32_t p : tab) {
        if (p < 0) return fail(CJ_ERR_ARG, "cj_attn_scores: negative page in the table");
        maxpg = std::max(maxpg, p);
    }
    if (!in_buffer(dptr(kcache), (((int64_t)maxpg + 1) * n_kv * 64) * head_dim * 2))
        return fail(CJ_ERR_ARG, "cj_attn_scores: page %d outside the K plane", maxpg);
    cj_attn_args a{};
    a.part = (float *)dptr(scores); a.q = (const float *)dptr(q); a.kc = (const uint16_t *)dptr(kcache);
    a.pgtab = (const int32_t *)dptr(pgtab); a.n_q = n_q; a.n_kv = n_kv; a.head_dim = head_dim; a.pg_base = pg_base;
    a.pg_n = (int32_t)pages; a.count = count; a.from = from; a.scale = scale; a.splits = count;   // the row stride
    char name[64];
    snprintf(name, sizeof name, "cj_attn_scores_h%d", head_dim);
    return launch2(name, (uint32_t)((count + 255) / 256), (uint32_t)n_q, 256, 0, a);
}

int32_t cj_moe_route(int64_t sel, int64_t weights, int64_t logits, int32_t rows, int32_t n_experts, int32_t n_used, int32_t norm_topk,
                     float w_scale, int64_t status) {
    if (rows <= 0 || n_experts <= 0 || n_experts > 256 || n_used <= 0 || n_used > n_experts || n_used > 16 ||
        !in_buffer(dptr(logits), (int64_t)rows * n_experts * 4) || !in_buffer(dptr(sel), (int64_t)rows * n_used * 4) ||
        !in_buffer(dptr(weights), (int64_t)rows * n_used * 4) || (status && !in_buffer(dptr(status), 4)))
        return fail(CJ_ERR_ARG, "cj_moe_route: rows %d experts %d used %d", rows, n_experts, n_used);
    cj_route_args a{(const float *)dptr(logits), (int32_t *)dptr(sel), (float *)dptr(weights), n_experts, n_used, norm_topk, rows,
                    w_scale, 0, status ? (int32_t *)dptr(status) : nullptr};
    return launch("cj_moe_route", (uint32_t)rows, 64, 0, a);
}

}  // extern "C"
