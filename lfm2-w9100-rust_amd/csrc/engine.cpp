// engine.cpp -- host runtime of the MI355X LFM2 Q6_K token loop behind the C
// ABI in include/lfm_hip.h.
//
// It replaces the reference's GpuEngine + resident graph + Vulkan runtime
// (Amidwestnoob/lfm2-w9100-rust engine/src/gpu_lfm.rs:23-245,
// engine/src/gpu_lfm/resident_graph.rs:4-602, engine/src/vulkan*.rs) with:
//   * one HIP stream per engine (default priority), all work in stream order;
//   * kernels from a gfx950 code object launched with hipModuleLaunchKernel;
//   * two captured hipGraphs: the layer stack + prompt advance (prefill by
//     decode steps) and the layer stack + head/argmax/feedback (decode step),
//     both reading token and position from device memory, so a decode run is
//     graph replays with no host round trip per token.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/lfm_hip.h"
#include "host_err.h"
#include "kargs.h"
#include "launch_host.h"

// ------------------------------------------------------------------ errors
static thread_local std::string g_err;

int lfm_vfail(int code, const char *fmt, va_list ap)
{
    char buf[1024];
    vsnprintf(buf, sizeof(buf), fmt, ap);
    g_err = buf;
    return code;
}

#define HIPCHK(call)                                                                          \
    do {                                                                                      \
        hipError_t _e = (call);                                                               \
        if (_e != hipSuccess)                                                                 \
            return fail(LFM_EDEVICE, "%s failed: %s (%s:%d)", #call, hipGetErrorString(_e),   \
                        __FILE__, __LINE__);                                                  \
    } while (0)

#define RC(call)                                                                              \
    do {                                                                                      \
        int _rc = (call);                                                                     \
        if (_rc != LFM_OK)                                                                    \
            return _rc;                                                                       \
    } while (0)

extern "C" const char *lfm_last_error(void) { return g_err.c_str(); }
extern "C" const char *lfm_version(void) { return "lfm2-mi355x 0.1 (gfx950)"; }

extern "C" int lfm_device_count(int *count)
{
    if (!count)
        return fail(LFM_EINVAL, "count is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = e == hipSuccess ? n : 0;
    return LFM_OK;
}

extern "C" int lfm_device_mem_info(int device, uint64_t *free_bytes, uint64_t *total_bytes)
{
    if (!free_bytes || !total_bytes)
        return fail(LFM_EINVAL, "null argument");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(LFM_EDEVICE, "no HIP device available");
    if (device < 0 || device >= n)
        return fail(LFM_EINVAL, "device %d out of range (%d devices)", device, n);
    HIPCHK(hipSetDevice(device));
    size_t free_b = 0, total_b = 0;
    HIPCHK(hipMemGetInfo(&free_b, &total_b));
    *free_bytes = free_b;
    *total_bytes = total_b;
    return LFM_OK;
}

// ------------------------------------------------------------------ kernels
// Launch shape of a decode matvec kernel: waves per workgroup (4 or 16, the
// kernel variant) and target rows (work items) per wave, which set the grid.
struct Shape {
    hipFunction_t f4 = nullptr, f16 = nullptr;
    hipFunction_t f4e = nullptr, f16e = nullptr; // embedding-input variants (first layer)
    uint32_t nw = 4, rpw = 1;
    hipFunction_t fn() const { return nw == 16 ? f16 : f4; }
    hipFunction_t fn(bool embed) const
    {
        return embed && f4e ? (nw == 16 ? f16e : f4e) : fn();
    }
    uint32_t threads() const { return 64 * nw; }
    uint32_t grid(uint32_t items) const
    {
        const uint32_t per = nw * rpw;
        return std::max(1u, (items + per - 1) / per);
    }
};

struct Kernels {
    hipModule_t mod = nullptr, pmod = nullptr;
    hipFunction_t split_rows, split_rows_ext, gemm_q6, conv_prefill, rope_kv_prefill, attn_prefill,
        gemm_swiglu, gemm_q6_t32, gemm_q6_t32n1, gemm_swiglu_t32, gemm_reduce, reduce_combine, attn_merge_split, router_small, router_mfma, router_split, route_topk, route_group, combine_prefill, embed_rows,
        tile_pack, gemm_q6_n64, gemm_q6_x, gemm_swiglu_x, gemm_q6_t32x, gemm_swiglu_t32x, tile_h16, gemm_h16,
        gemm_h16_n64, gemm_swiglu_h16;
    hipFunction_t matvec_long, attn, attn_merge, router, moe_down, argmax, argmax_final, advance,
        dequant, copy, matvec_route, gateup_f, conv_mixer, conv_mixer_r;
    Shape matvec, conv, qkv, gateup, head;
    DevState *idle_st = nullptr; // zeroed state for op-level matvecs (never halted)
};

// Shapes measured best on MI355X for the LFM2-8B widths; LFM_DECODE_SHAPES
// ("matvec=4x1,conv=4x1,qkv=4x1,gateup=4x2,head=4x16") overrides them.
static void set_shapes(Kernels *k)
{
    k->matvec.nw = 4, k->matvec.rpw = 1;
    k->conv.nw = 4, k->conv.rpw = 1;
    k->qkv.nw = 4, k->qkv.rpw = 1;
    k->gateup.nw = 4, k->gateup.rpw = 2;
    k->head.nw = 4, k->head.rpw = 16;
    const char *env = getenv("LFM_DECODE_SHAPES");
    if (!env)
        return;
    struct {
        const char *name;
        Shape *s;
    } tab[] = {{"matvec", &k->matvec}, {"conv", &k->conv}, {"qkv", &k->qkv},
               {"gateup", &k->gateup}, {"head", &k->head}};
    std::string spec(env);
    size_t pos = 0;
    while (pos < spec.size()) {
        size_t end = spec.find(',', pos);
        if (end == std::string::npos)
            end = spec.size();
        const std::string item = spec.substr(pos, end - pos);
        const size_t eq = item.find('='), x = item.find('x');
        if (eq != std::string::npos && x != std::string::npos && x > eq)
            for (auto &t : tab)
                if (item.compare(0, eq, t.name) == 0) {
                    const uint32_t nw = (uint32_t)atoi(item.c_str() + eq + 1);
                    const uint32_t rpw = (uint32_t)atoi(item.c_str() + x + 1);
                    if ((nw == 4 || nw == 16) && rpw >= 1 && rpw <= 64)
                        t.s->nw = nw, t.s->rpw = rpw;
                }
        pos = end + 1;
    }
}

static std::mutex g_kmu;
static std::unordered_map<int, Kernels *> g_kernels;

static std::string code_object_path()
{
    const char *env = getenv("LFM_KERNELS");
    if (env && *env)
        return env;
    Dl_info info;
    if (dladdr((void *)&lfm_version, &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        size_t slash = p.rfind('/');
        std::string dir = slash == std::string::npos ? "." : p.substr(0, slash);
        return dir + "/lfm_kernels.hsaco";
    }
    return "lfm_kernels.hsaco";
}

// The prefill kernels live in a second code object next to the first.
static std::string prefill_object_path()
{
    std::string p = code_object_path();
    const size_t slash = p.rfind('/');
    return (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) + "/lfm_prefill.hsaco";
}

// Loads the code object on the current device (once per device).
static int get_kernels(Kernels **out)
{
    int dev = 0;
    HIPCHK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_kmu);
    auto it = g_kernels.find(dev);
    if (it != g_kernels.end()) {
        *out = it->second;
        return LFM_OK;
    }
    Kernels *k = new Kernels();
    std::string path = code_object_path();
    hipError_t e = hipModuleLoad(&k->mod, path.c_str());
    if (e != hipSuccess) {
        delete k;
        return fail(LFM_EDEVICE, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
    }
    struct {
        hipFunction_t *f;
        const char *name;
    } fns[] = {{&k->matvec.f4, "k_q6_matvec4"},   {&k->matvec.f16, "k_q6_matvec16"},
               {&k->matvec_long, "k_q6_matvec_long"}, {&k->conv.f4, "k_conv_inproj4"},
               {&k->conv.f16, "k_conv_inproj16"}, {&k->qkv.f4, "k_qkv4"},
               {&k->qkv.f16, "k_qkv16"},          {&k->attn, "k_attn"},
               {&k->conv.f4e, "k_conv_inproj4e"}, {&k->conv.f16e, "k_conv_inproj16e"},
               {&k->qkv.f4e, "k_qkv4e"},          {&k->qkv.f16e, "k_qkv16e"},
               {&k->attn_merge, "k_attn_merge"},  {&k->router, "k_router"},
               {&k->gateup.f4, "k_gateup4"},      {&k->gateup.f16, "k_gateup16"},
               {&k->moe_down, "k_moe_down"},      {&k->head.f4, "k_head4"},
               {&k->head.f16, "k_head16"},        {&k->argmax, "k_argmax"},
               {&k->argmax_final, "k_argmax_final"}, {&k->advance, "k_advance"},
               {&k->dequant, "k_q6_dequant"},    {&k->copy, "k_copy"},
               {&k->matvec_route, "k_q6_matvec_route"}, {&k->gateup_f, "k_gateup8f"},
               {&k->conv_mixer, "k_conv_mixer"},  {&k->conv_mixer_r, "k_conv_mixer_r"}};
    for (auto &f : fns) {
        e = hipModuleGetFunction(f.f, k->mod, f.name);
        if (e != hipSuccess) {
            (void)hipModuleUnload(k->mod);
            delete k;
            return fail(LFM_EDEVICE, "hipModuleGetFunction(%s): %s", f.name, hipGetErrorString(e));
        }
    }
    const std::string ppath = prefill_object_path();
    e = hipModuleLoad(&k->pmod, ppath.c_str());
    if (e != hipSuccess) {
        (void)hipModuleUnload(k->mod);
        delete k;
        return fail(LFM_EDEVICE, "hipModuleLoad(%s): %s", ppath.c_str(), hipGetErrorString(e));
    }
    struct {
        hipFunction_t *f;
        const char *name;
    } pfns[] = {{&k->split_rows, "k_split_rows"},       {&k->split_rows_ext, "k_split_rows_ext"},
                {&k->gemm_q6, "k_gemm_q6"},
                {&k->conv_prefill, "k_conv_prefill"},
                {&k->rope_kv_prefill, "k_rope_kv_prefill"}, {&k->attn_prefill, "k_attn_prefill"},
                {&k->gemm_swiglu, "k_gemm_q6_swiglu"}, {&k->router_mfma, "k_router_mfma"}, {&k->router_split, "k_router_split"},
                {&k->route_topk, "k_route_topk"},       {&k->route_group, "k_route_group"},
                {&k->combine_prefill, "k_combine_prefill"}, {&k->gemm_reduce, "k_gemm_reduce"},
                {&k->gemm_q6_t32, "k_gemm_q6_t32"},     {&k->gemm_swiglu_t32, "k_gemm_q6_swiglu_t32"},
                {&k->gemm_q6_t32n1, "k_gemm_q6_t32n1"},
                {&k->attn_merge_split, "k_attn_merge_split"}, {&k->reduce_combine, "k_reduce_combine"}, {&k->router_small, "k_router_prefill_small"},
                {&k->embed_rows, "k_embed_rows"}, {&k->tile_pack, "k_q6_tile_pack"},
                {&k->gemm_q6_n64, "k_gemm_q6_n64"}, {&k->gemm_q6_x, "k_gemm_q6_x"},
                {&k->gemm_swiglu_x, "k_gemm_q6_swiglu_x"}, {&k->gemm_q6_t32x, "k_gemm_q6_t32x"},
                {&k->gemm_swiglu_t32x, "k_gemm_q6_swiglu_t32x"}, {&k->tile_h16, "k_q6_tile_h16"},
                {&k->gemm_h16, "k_gemm_h16"}, {&k->gemm_h16_n64, "k_gemm_h16_n64"},
                {&k->gemm_swiglu_h16, "k_gemm_swiglu_h16"}};
    for (auto &f : pfns) {
        e = hipModuleGetFunction(f.f, k->pmod, f.name);
        if (e != hipSuccess) {
            (void)hipModuleUnload(k->mod);
            (void)hipModuleUnload(k->pmod);
            delete k;
            return fail(LFM_EDEVICE, "hipModuleGetFunction(%s): %s", f.name, hipGetErrorString(e));
        }
    }
    set_shapes(k);
    if (hipMalloc(&k->idle_st, sizeof(DevState)) != hipSuccess ||
        hipMemset(k->idle_st, 0, sizeof(DevState)) != hipSuccess) {
        if (k->idle_st)
            (void)hipFree(k->idle_st);
        (void)hipModuleUnload(k->mod);
        (void)hipModuleUnload(k->pmod);
        delete k;
        return fail(LFM_EDEVICE, "device state allocation failed");
    }
    const int src = lfm_noalloc_setup(dev);
    if (src != LFM_OK) {
        (void)hipFree(k->idle_st);
        (void)hipModuleUnload(k->mod);
        (void)hipModuleUnload(k->pmod);
        delete k;
        return src;
    }
    g_kernels[dev] = k;
    *out = k;
    return LFM_OK;
}

template <typename A>
static int launch_t(hipFunction_t f, dim3 grid, uint32_t threads, uint32_t smem, hipStream_t s,
                    const A &args)
{
    void *params[] = {(void *)&args};
    HIPCHK(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, threads, 1, 1, smem, s, params, nullptr));
    return LFM_OK;
}

template <typename A>
static int launch(hipFunction_t f, dim3 grid, uint32_t smem, hipStream_t s, const A &args)
{
    return launch_t(f, grid, 256, smem, s, args);
}

// A decode matvec kernel over `items` work items, in its tuned shape.
template <typename A>
static int launch_shape(const Shape &sh, uint32_t items, hipStream_t s, const A &args)
{
    return launch_t(sh.fn(), dim3(sh.grid(items)), sh.threads(), 0, s, args);
}

// Mixer kernels: the first layer of a step reads the token's embedding row.
template <typename A>
static int launch_mixer(const Shape &sh, uint32_t items, hipStream_t s, const A &args)
{
    return launch_t(sh.fn(args.src.embed != 0), dim3(sh.grid(items)), sh.threads(), 0, s, args);
}

// ------------------------------------------------------------------ Q6_K layout
extern "C" size_t lfm_q6k_nbytes(uint64_t rows, uint64_t in_dim) { return rows * (in_dim / 256) * 210; }

// GGUF block_q6_K (ql[128] qh[64] scales[16] d[2]) -> four planes (kargs.h).
static void pack_blocks(const uint8_t *raw, uint64_t nblk, uint8_t *out)
{
    uint8_t *ql = out, *qh = out + nblk * 128, *sc = out + nblk * 192, *dd = out + nblk * 208;
    for (uint64_t b = 0; b < nblk; ++b) {
        const uint8_t *r = raw + b * 210;
        for (int c = 0; c < 8; ++c) {
            const int h = c >> 2, l0 = (c & 3) * 8;
            memcpy(ql + b * 128 + c * 16, r + h * 64 + l0, 8);
            memcpy(ql + b * 128 + c * 16 + 8, r + h * 64 + 32 + l0, 8);
        }
        memcpy(qh + b * 64, r + 128, 64);
        for (int p = 0; p < 4; ++p)
            for (int s = 0; s < 4; ++s)
                sc[b * 16 + p * 4 + s] = r[192 + (p >> 1) * 8 + (p & 1) + 2 * s];
        dd[b * 2] = r[208];
        dd[b * 2 + 1] = r[209];
    }
}

static void unpack_blocks(const uint8_t *packed, uint64_t nblk, uint8_t *raw)
{
    const uint8_t *ql = packed, *qh = packed + nblk * 128, *sc = packed + nblk * 192,
                  *dd = packed + nblk * 208;
    for (uint64_t b = 0; b < nblk; ++b) {
        uint8_t *r = raw + b * 210;
        for (int c = 0; c < 8; ++c) {
            const int h = c >> 2, l0 = (c & 3) * 8;
            memcpy(r + h * 64 + l0, ql + b * 128 + c * 16, 8);
            memcpy(r + h * 64 + 32 + l0, ql + b * 128 + c * 16 + 8, 8);
        }
        memcpy(r + 128, qh + b * 64, 64);
        for (int p = 0; p < 4; ++p)
            for (int s = 0; s < 4; ++s)
                r[192 + (p >> 1) * 8 + (p & 1) + 2 * s] = sc[b * 16 + p * 4 + s];
        r[208] = dd[b * 2];
        r[209] = dd[b * 2 + 1];
    }
}

extern "C" int lfm_q6k_pack(const void *raw, uint64_t rows, uint64_t in_dim, void *packed)
{
    if (!raw || !packed || in_dim == 0 || in_dim % 256)
        return fail(LFM_EINVAL, "lfm_q6k_pack: in_dim must be a positive multiple of 256");
    pack_blocks((const uint8_t *)raw, rows * (in_dim / 256), (uint8_t *)packed);
    return LFM_OK;
}

extern "C" int lfm_q6k_unpack(const void *packed, uint64_t rows, uint64_t in_dim, void *raw)
{
    if (!raw || !packed || in_dim == 0 || in_dim % 256)
        return fail(LFM_EINVAL, "lfm_q6k_unpack: in_dim must be a positive multiple of 256");
    unpack_blocks((const uint8_t *)packed, rows * (in_dim / 256), (uint8_t *)raw);
    return LFM_OK;
}

// ------------------------------------------------------------------ device buffers
extern "C" int lfm_dev_alloc(size_t nbytes, void **ptr)
{
    if (!ptr)
        return fail(LFM_EINVAL, "ptr is null");
    HIPCHK(hipMalloc(ptr, nbytes ? nbytes : 1));
    return LFM_OK;
}
extern "C" int lfm_dev_free(void *ptr)
{
    HIPCHK(hipFree(ptr));
    return LFM_OK;
}
extern "C" int lfm_memcpy_htod(void *dst, const void *src, size_t n)
{
    HIPCHK(hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
    // from pageable memory the copy may still be in flight when hipMemcpy
    // returns: wait, so that work on any stream sees the data
    HIPCHK(hipDeviceSynchronize());
    return LFM_OK;
}
extern "C" int lfm_memcpy_dtoh(void *dst, const void *src, size_t n)
{
    HIPCHK(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost));
    return LFM_OK;
}
extern "C" int lfm_dev_synchronize(void)
{
    HIPCHK(hipDeviceSynchronize());
    return LFM_OK;
}

// Matvec input widths: 1..32 blocks (256..8192 inputs).
static int matvec_check(uint32_t nb)
{
    if (nb == 0 || nb > 32)
        return fail(LFM_EINVAL, "Q6_K matvec supports 256..8192 inputs (got %u blocks)", nb);
    return LFM_OK;
}

// Launches y = W x (mode 0) or y += W x (mode 1): the one-wave-per-row kernel for
// rows of up to 8 blocks, the 16-wave split-row kernel for longer rows.
static int launch_matvec(Kernels *K, MatvecArgs &m, hipStream_t s)
{
    if (!m.st)
        m.st = K->idle_st;
    RC(matvec_check(m.w.nb));
    if (m.w.nb <= 8)
        return launch_shape(K->matvec, m.w.rows, s, m);
    const uint32_t grid = (m.w.rows + LONG_ROWS - 1) / LONG_ROWS;
    if (grid > 0x7FFFFFFFu)
        return fail(LFM_EINVAL, "too many rows");
    return launch_t(K->matvec_long, dim3(grid), 1024, 0, s, m);
}

static Q6T q6view(const void *dev, uint64_t rows, uint64_t in_dim)
{
    Q6T t;
    t.base = (const uint8_t *)dev;
    t.rows = (uint32_t)rows;
    t.nb = (uint32_t)(in_dim / 256);
    return t;
}

// The prefill GEMMs' copy of a row-major Q6_K matrix of src.rows / group_rows
// slices in 32-row tiles (layout at Q6Tiles), written by k_q6_tile_pack on s.  The
// kernel's wide-scale flag sits in the same allocation, past the tiles, so that
// packs on other streams or threads (other engines, lfm_q6k_gemm) never share it.
static int make_tiles(Kernels *K, hipStream_t s, const Q6T &src, uint32_t group_rows, void **dev, Q6Tiles *out)
{
    *dev = nullptr;
    if (group_rows == 0 || src.rows % group_rows)
        return fail(LFM_EINVAL, "tile copy: %u rows are not whole slices of %u", src.rows, group_rows);
    const uint32_t gtiles = (group_rows + 31) / 32;
    const uint64_t tiles = (uint64_t)(src.rows / group_rows) * gtiles, ntb = tiles * src.nb;
    if (ntb > 0x7FFFFFFFull)
        return fail(LFM_EINVAL, "tile copy: %llu tile-blocks exceed the grid", (unsigned long long)ntb);
    const uint64_t bytes = ntb * TILE_BYTES, flag_at = (bytes + 255) / 256 * 256;
    if (hipMalloc(dev, flag_at + 256) != hipSuccess) {
        *dev = nullptr;
        return fail(LFM_EDEVICE, "tile copy: device allocation of %llu bytes failed",
                    (unsigned long long)(flag_at + 256));
    }
    uint32_t *flag = reinterpret_cast<uint32_t *>((uint8_t *)*dev + flag_at);
    TilePackArgs a{src, (uint8_t *)*dev, group_rows, gtiles, (uint32_t)tiles, flag};
    uint32_t wide = 0;
    int rc = hipMemsetAsync(flag, 0, 4, s) == hipSuccess ? LFM_OK : fail(LFM_EDEVICE, "tile copy: flag reset");
    if (rc == LFM_OK)
        rc = launch_t(K->tile_pack, dim3((uint32_t)ntb), 64, 0, s, a);
    if (rc == LFM_OK && (hipMemcpyAsync(&wide, flag, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
                         hipStreamSynchronize(s) != hipSuccess))
        rc = fail(LFM_EDEVICE, "tile copy: flag read");
    if (rc != LFM_OK) {
        (void)hipFree(*dev);
        *dev = nullptr;
        return rc;
    }
    *out = Q6Tiles{(const uint8_t *)*dev, (uint32_t)tiles, src.nb, gtiles, group_rows, wide ? 1u : 0u, nullptr};
    return LFM_OK;
}

// The binary16 fragment copy of a tile copy (kargs.h TILE_H16), which the large-call
// GEMMs read instead of decoding Q6_K: made when every scale of the tensor lies
// within [-64, 64] (binary16 then holds its weights exactly) unless LFM_PREFILL_H16=0.
// 16 KB per tile-block (2.4 times the Q6_K bytes).  Without it (wide scales, the
// variable set, or no device memory for it) t->h16 stays null and those calls
// decode Q6_K in registers as the small calls do.
static bool h16_wanted()
{
    const char *v = getenv("LFM_PREFILL_H16");
    return !(v && strcmp(v, "0") == 0);
}

static bool ends_with(const std::string &s, const char *suffix)
{
    const size_t m = strlen(suffix);
    return s.size() >= m && s.compare(s.size() - m, m, suffix) == 0;
}

static int make_h16(Kernels *K, hipStream_t s, Q6Tiles *t, void **dev)
{
    *dev = nullptr;
    t->h16 = nullptr;
    if (t->wide || !h16_wanted())
        return LFM_OK;
    const uint64_t ntb = (uint64_t)t->tiles * t->nb;
    if (hipMalloc(dev, ntb * TILE_H16) != hipSuccess) {
        (void)hipGetLastError(); // out of device memory: keep the Q6_K kernels
        *dev = nullptr;
        return LFM_OK;
    }
    TileH16Args a{*t, (uint8_t *)*dev};
    const int rc = launch_t(K->tile_h16, dim3((uint32_t)ntb), 64, 0, s, a);
    if (rc != LFM_OK) {
        (void)hipFree(*dev);
        *dev = nullptr;
        return rc;
    }
    t->h16 = (const uint8_t *)*dev;
    return LFM_OK;
}

static int check_q6_args(const void *packed, uint64_t rows, uint64_t in_dim)
{
    if (!packed || rows == 0 || rows > 0xFFFFFFFFull || in_dim == 0 || in_dim % 256)
        return fail(LFM_EINVAL, "Q6_K tensor: rows must be 1..2^32-1, in_dim a multiple of 256");
    return LFM_OK;
}

extern "C" int lfm_q6k_dequant(const void *packed, uint64_t rows, uint64_t in_dim, float *out,
                               void *stream)
{
    RC(check_q6_args(packed, rows, in_dim));
    Kernels *K;
    RC(get_kernels(&K));
    DequantArgs a;
    a.w = q6view(packed, rows, in_dim);
    a.out = out;
    a.in_dim = (uint32_t)in_dim;
    const uint64_t units = rows * (in_dim / 256) * 8;
    const uint32_t grid = (uint32_t)std::min<uint64_t>((units + 255) / 256, 65535);
    RC(launch(K->dequant, dim3(grid), 0, (hipStream_t)stream, a));
    HIPCHK(hipStreamSynchronize((hipStream_t)stream));
    return LFM_OK;
}

static int matvec_args(const void *packed, uint64_t rows, uint64_t in_dim, const float *x, float *y,
                       MatvecArgs *a)
{
    RC(check_q6_args(packed, rows, in_dim));
    memset(a, 0, sizeof(*a));
    a->w = q6view(packed, rows, in_dim);
    a->src.x = x;
    a->y = y;
    a->in_dim = (uint32_t)in_dim;
    a->mode = 0;
    return matvec_check(a->w.nb);
}

extern "C" int lfm_q6k_matvec(const void *packed, uint64_t rows, uint64_t in_dim, const float *x,
                              float *y, void *stream)
{
    MatvecArgs a;
    RC(matvec_args(packed, rows, in_dim, x, y, &a));
    Kernels *K;
    RC(get_kernels(&K));
    RC(launch_matvec(K, a, (hipStream_t)stream));
    HIPCHK(hipStreamSynchronize((hipStream_t)stream));
    return LFM_OK;
}

extern "C" int lfm_copy_time(uint64_t bytes, uint32_t reps, float *us_per_copy)
{
    if (bytes < 16 || bytes % 16 || reps == 0 || !us_per_copy)
        return fail(LFM_EINVAL, "copy: bytes must be a positive multiple of 16, reps positive");
    Kernels *K;
    RC(get_kernels(&K));
    void *src = nullptr, *dst = nullptr;
    HIPCHK(hipMalloc(&src, bytes));
    if (hipMalloc(&dst, bytes) != hipSuccess) {
        (void)hipFree(src);
        return fail(LFM_EDEVICE, "copy: allocation of %llu bytes failed", (unsigned long long)bytes);
    }
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = LFM_OK;
    float ms = 0.f;
    CopyArgs a{(const uint4 *)src, (uint4 *)dst, bytes / 16};
    const uint32_t grid = 2048;
    if (hipMemset(src, 1, bytes) != hipSuccess || hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
        rc = fail(LFM_EDEVICE, "copy: setup failed");
    if (rc == LFM_OK)
        rc = launch(K->copy, dim3(grid), 0, s, a); // warm
    if (rc == LFM_OK && hipEventRecord(e0, s) != hipSuccess)
        rc = fail(LFM_EDEVICE, "copy: event record failed");
    for (uint32_t i = 0; i < reps && rc == LFM_OK; ++i)
        rc = launch(K->copy, dim3(grid), 0, s, a);
    if (rc == LFM_OK && (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                         hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
        rc = fail(LFM_EDEVICE, "copy: timing failed");
    if (e0)
        (void)hipEventDestroy(e0);
    if (e1)
        (void)hipEventDestroy(e1);
    if (s)
        (void)hipStreamDestroy(s);
    (void)hipFree(src);
    (void)hipFree(dst);
    if (rc == LFM_OK)
        *us_per_copy = ms * 1000.f / (float)reps;
    return rc;
}

extern "C" int lfm_q6k_matvec_time(const void *packed, uint32_t ncopies, uint64_t rows,
                                   uint64_t in_dim, const float *x, float *y, uint32_t iters,
                                   float *ms)
{
    if (ncopies == 0 || iters == 0 || !ms)
        return fail(LFM_EINVAL, "ncopies, iters must be positive and ms non-null");
    MatvecArgs a;
    RC(matvec_args(packed, rows, in_dim, x, y, &a));
    Kernels *K;
    RC(get_kernels(&K));
    hipStream_t s;
    HIPCHK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    const size_t sz = lfm_q6k_nbytes(rows, in_dim);
    for (uint32_t i = 0; i < std::min(iters, ncopies); ++i) { // warm the code path
        a.w.base = (const uint8_t *)packed + (size_t)(i % ncopies) * sz;
        RC(launch_matvec(K, a, s));
    }
    HIPCHK(hipEventRecord(e0, s));
    for (uint32_t i = 0; i < iters; ++i) {
        a.w.base = (const uint8_t *)packed + (size_t)(i % ncopies) * sz;
        RC(launch_matvec(K, a, s));
    }
    HIPCHK(hipEventRecord(e1, s));
    HIPCHK(hipEventSynchronize(e1));
    float total = 0.f;
    HIPCHK(hipEventElapsedTime(&total, e0, e1));
    *ms = total / (float)iters;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipStreamDestroy(s);
    return LFM_OK;
}

// ------------------------------------------------------------------ MFMA GEMM
#define DECODE_WINDOW 32u // lfm_decode_run: replays per window (two windows queued at most)
#define GEMM_ROWS 256   // weight rows per GEMM workgroup
#define GEMM_TOKENS 128 // token columns per GEMM workgroup
#define GEMM_THREADS 256 // 4 waves of 64 weight rows each
static dim3 gemm_grid(uint32_t rows, uint32_t ntok, uint32_t nz, uint32_t rows_per_wg = GEMM_ROWS,
                      uint32_t tokens_per_wg = GEMM_TOKENS)
{
    return dim3((rows + rows_per_wg - 1) / rows_per_wg, (ntok + tokens_per_wg - 1) / tokens_per_wg, nz);
}

#define GEMM_PART_BYTES ((size_t)64 << 20) // split-K partial sums (prefill scratch)
#define GEMM_PART_SOFT ((size_t)1600000) // small calls' partial sums, floats (6.4 MB)
#define GEMM_N64_BELOW 512u // two 128-token workgroups per CU on 256 CUs

// Launches the matrix-core GEMM g (pair: gate + up + SwiGLU) over T tokens and nz
// groups.  Up to one 128-token tile (T <= 128, as in 64-token chunked prefill,
// about 8 tokens per expert) the kernels with 32-token tiles run, the grid is
// then mostly the weight-row tiles and each workgroup's K loop is a chain of
// dependent stages, so K is split into slices (about 1024 workgroups, each slice
// at least one Q6_K block, the partials within `part_cap` floats of `part` and
// within GEMM_PART_SOFT floats) and
// k_gemm_reduce adds the slices in order.  part_rows: output rows the GEMM can
// write (T, or 4T for expert slots); n_used: ranks per token of the expert slots.
// `deferred` (ungrouped, non-pair calls): with a K split the reduce is left to the
// caller, which gets the slice count there (1: the kernel wrote c itself; S > 1: the
// S slices of part, each part_rows x zrows).
// Router partials for the next FFN (ungrouped, non-pair, accumulating calls): with
// a K split the reduce also leaves them (GemmReduceArgs) and *router_done is set.
struct RouterPart {
    const float *norm, *w; // the FFN's RMSNorm weight and router rows [n_expert][zrows]
    float *rpart, *rss;
    uint32_t n_expert;
    uint32_t *counts; // nullable: zeroed by the reduce (the next split counts into it)
};

static int launch_gemm(Kernels *K, hipStream_t s, GemmArgs g, bool pair, uint32_t T, uint32_t nz,
                       uint32_t part_rows, uint32_t n_used, float *part, size_t part_cap, uint64_t *dispatches,
                       const CombinePrefillArgs *combine = nullptr, bool *combined = nullptr,
                       uint32_t *deferred = nullptr, const RouterPart *router = nullptr, bool *router_done = nullptr,
                       ReduceCombineArgs *defer_combine = nullptr)
{
    if (router_done)
        *router_done = false;
    if (combined)
        *combined = false;
    const bool small = T <= GEMM_TOKENS;
    // weights with scales outside [-64, 64] take the split-scale kernels (one 32-row
    // tile per wave for small single-weight calls, 64 tokens per large workgroup)
    const bool exact = g.w.wide || (pair && g.w2.wide);
    // small ungrouped projections of up to 3072 rows (q/k/v, the out projections):
    // one 32-row tile per wave
    const bool one_tile = small && !pair && (exact || (nz == 1 && g.zrows <= 3072));
    // large single-weight calls whose 128-token grid would not give each CU two
    // workgroups (few row tiles: the 2048- and 3072-row projections) take 64 tokens
    // per workgroup
    const dim3 g128 = gemm_grid(g.zrows, T, nz, GEMM_ROWS, GEMM_TOKENS);
    const bool n64 = !small && !pair && (exact || (uint64_t)g128.x * g128.y * g128.z < GEMM_N64_BELOW);
    const bool t64 = n64 || (!small && pair && exact);
    // large calls over weights with a binary16 fragment copy read it (no decode)
    const bool h16 = !small && !exact && g.w.h16 && (!pair || g.w2.h16);
    dim3 grid = gemm_grid(g.zrows, T, nz, pair || one_tile ? GEMM_ROWS / 2 : GEMM_ROWS,
                          small ? 32 : t64 ? GEMM_TOKENS / 2 : GEMM_TOKENS);
    uint32_t S = 1;
    if (part && small) {
        const uint32_t wgs = grid.x * grid.y * grid.z;
        const size_t per = (size_t)(pair ? 2 : 1) * part_rows * g.zrows;
        S = std::min<uint32_t>(std::max<uint32_t>(1, 1024 / wgs), g.w.nb);
        // and at most GEMM_PART_SOFT floats of partial sums: past that, writing and
        // adding them costs more than the wider grid gains (the 6144-row in_proj at
        // four slices, the dense gate/up pair unsplit, the dense down at twelve)
        S = (uint32_t)std::max<size_t>(1, std::min<size_t>(S, std::min<size_t>(part_cap, GEMM_PART_SOFT) / per));
        if (g.y_hi) // the split output is formed in the epilogue from whole sums
            S = 1;
    }
    hipFunction_t f = small ? (pair ? (exact ? K->gemm_swiglu_t32x : K->gemm_swiglu_t32)
                                    : one_tile ? (exact ? K->gemm_q6_t32x : K->gemm_q6_t32n1) : K->gemm_q6_t32)
                    : h16 ? (pair ? K->gemm_swiglu_h16 : n64 ? K->gemm_h16_n64 : K->gemm_h16)
                            : (pair ? (exact ? K->gemm_swiglu_x : K->gemm_swiglu)
                                    : n64 ? (exact ? K->gemm_q6_x : K->gemm_q6_n64) : K->gemm_q6);
    if (deferred)
        *deferred = S;
    if (S == 1) {
        RC(launch_t(f, grid, GEMM_THREADS, 0, s, g));
        *dispatches += 1;
        return LFM_OK;
    }
    g.part = part;
    g.ksplit = S;
    g.nz = nz;
    g.part_rows = part_rows;
    grid.z = nz * S;
    RC(launch_t(f, grid, GEMM_THREADS, 0, s, g));
    if (deferred) {
        *dispatches += 1;
        return LFM_OK;
    }
    if (combine) { // grouped down projection: slices and the rank combine in one pass
        ReduceCombineArgs rc{part, combine->wsel, combine->x, S, combine->T, combine->dim, combine->n_used};
        *combined = true;
        if (defer_combine) { // the caller's next split applies it
            *defer_combine = rc;
            *dispatches += 1;
            return LFM_OK;
        }
        RC(launch(K->reduce_combine, dim3((combine->dim + 255) / 256, combine->T), 0, s, rc));
    } else {
        GemmReduceArgs r{part, g.c, S, pair ? 1u : 0u, part_rows, g.zrows, g.ldc, g.col0, g.mode, n_used,
                         nullptr, nullptr, nullptr, nullptr, 0, nullptr};
        if (router && !pair && nz == 1 && g.zrows % 256 == 0 && router->n_expert <= 64) {
            r.rnorm = router->norm;
            r.rw = router->w;
            r.rpart = router->rpart;
            r.rss = router->rss;
            r.n_expert = router->n_expert;
            r.counts = router->counts;
            if (router_done)
                *router_done = true;
        }
        RC(launch(K->gemm_reduce, dim3((g.zrows + 255) / 256, part_rows), 0, s, r));
    }
    *dispatches += 2;
    return LFM_OK;
}

// Y[t][r] = sum_k W[r][k] X[t][k] for T token rows (prefill GEMM, op level).
extern "C" int lfm_q6k_gemm(const void *packed, uint64_t rows, uint64_t in_dim, const float *x,
                            uint32_t T, float *y, void *stream)
{
    RC(check_q6_args(packed, rows, in_dim));
    if (!x || !y || T == 0)
        return fail(LFM_EINVAL, "lfm_q6k_gemm: empty input");
    if (in_dim > 8192)
        return fail(LFM_EINVAL, "lfm_q6k_gemm: in_dim up to 8192");
    // the GEMM kernels address the binary16 activation copies (T rows, padded to 32
    // for small calls) with byte offsets below 2^31
    if (((uint64_t)T + 31) * in_dim * 2 > 0x7fffffffull)
        return fail(LFM_EINVAL, "lfm_q6k_gemm: (T + 31) x in_dim x 2 bytes must stay below 2 GiB");
    Kernels *K;
    RC(get_kernels(&K));
    hipStream_t s = (hipStream_t)stream;
    uint16_t *hi = nullptr, *lo = nullptr;
    float *scale = nullptr;
    // small calls (T <= GEMM_TOKENS) use the token-blocked layout, rows padded to 32
    const size_t hrows = T <= GEMM_TOKENS ? (T + 31) / 32 * 32 : T;
    HIPCHK(hipMalloc(&hi, hrows * in_dim * 2));
    HIPCHK(hipMalloc(&lo, hrows * in_dim * 2));
    HIPCHK(hipMalloc(&scale, (size_t)T * 4));
    float *bscale = nullptr; // small calls: the half-block scales of the blocked rows
    if (T <= GEMM_TOKENS && hipMalloc(&bscale, hrows * (in_dim / 128) * 4) != hipSuccess) {
        (void)hipFree(hi);
        (void)hipFree(lo);
        (void)hipFree(scale);
        return fail(LFM_EDEVICE, "lfm_q6k_gemm: scale allocation failed");
    }
    SplitArgs sa;
    memset(&sa, 0, sizeof(sa));
    sa.x = x;
    sa.hi = hi;
    sa.lo = lo;
    sa.scale = scale;
    sa.bscale = bscale;
    sa.T = T;
    sa.K = (uint32_t)in_dim;
    sa.mode = T <= GEMM_TOKENS ? SPLIT_BLOCKED : SPLIT_ROWMAJOR;
    int rc = launch(K->split_rows, dim3(T), 0, s, sa);
    GemmArgs ga;
    memset(&ga, 0, sizeof(ga));
    void *tiles = nullptr, *h16 = nullptr;
    if (rc == LFM_OK)
        rc = make_tiles(K, s, q6view(packed, rows, in_dim), (uint32_t)rows, &tiles, &ga.w);
    if (rc == LFM_OK && T > GEMM_TOKENS)
        rc = make_h16(K, s, &ga.w, &h16);
    ga.x_hi = hi;
    ga.x_lo = lo;
    ga.xscale = scale;
    ga.bscale = bscale;
    ga.ntok = T;
    ga.zrows = (uint32_t)rows;
    ga.c = y;
    ga.ldc = (uint32_t)rows;
    float *part = nullptr;
    size_t part_cap = 0;
    if (rc == LFM_OK && T <= GEMM_TOKENS) {
        part_cap = std::min<size_t>(GEMM_PART_BYTES / 4, (size_t)T * rows * (in_dim / 256));
        if (hipMalloc(&part, part_cap * 4) != hipSuccess)
            rc = fail(LFM_EDEVICE, "lfm_q6k_gemm: scratch allocation failed");
    }
    uint64_t nd = 0;
    if (rc == LFM_OK)
        rc = launch_gemm(K, s, ga, false, T, 1, T, 0, part, part_cap, &nd);
    if (rc == LFM_OK && hipStreamSynchronize(s) != hipSuccess)
        rc = fail(LFM_EDEVICE, "lfm_q6k_gemm: synchronize failed");
    (void)hipFree(hi);
    (void)hipFree(lo);
    (void)hipFree(scale);
    if (bscale)
        (void)hipFree(bscale);
    if (part)
        (void)hipFree(part);
    if (tiles)
        (void)hipFree(tiles);
    if (h16)
        (void)hipFree(h16);
    return rc;
}

uint32_t lfm_argmax_grid(uint32_t n)
{
    return std::max<uint32_t>(1, std::min<uint32_t>((n + 255) / 256, NOALLOC_ARGMAX_WGS));
}

int lfm_argmax_enqueue(const float *v, uint32_t n, DevState *st, float *partial, hipStream_t s)
{
    Kernels *K;
    RC(get_kernels(&K));
    const uint32_t grid = lfm_argmax_grid(n);
    ArgmaxArgs a{v, partial, n, st};
    FinalArgs f{partial, grid, nullptr, 0, st, nullptr};
    RC(launch(K->argmax, dim3(grid), 0, s, a));
    return launch(K->argmax_final, dim3(1), 0, s, f);
}

// Stand-alone argmax with a state block and partials allocated per call.
extern "C" int lfm_argmax(const float *v, uint32_t n, uint32_t *index, float *value)
{
    if (!v || n == 0 || !index)
        return fail(LFM_EINVAL, "lfm_argmax: empty input");
    Kernels *K;
    RC(get_kernels(&K));
    const uint32_t grid = lfm_argmax_grid(n);
    DevState *st = nullptr;
    float *partial = nullptr;
    HIPCHK(hipMalloc(&st, sizeof(DevState)));
    HIPCHK(hipMalloc(&partial, grid * 2 * sizeof(float)));
    DevState h;
    memset(&h, 0, sizeof(h));
    HIPCHK(hipMemcpy(st, &h, sizeof(h), hipMemcpyHostToDevice));
    int rc = lfm_argmax_enqueue(v, n, st, partial, nullptr);
    if (rc == LFM_OK) {
        HIPCHK(hipDeviceSynchronize());
        HIPCHK(hipMemcpy(&h, st, sizeof(h), hipMemcpyDeviceToHost));
        *index = h.last_token;
        if (value)
            *value = h.last_value;
    }
    (void)hipFree(st);
    (void)hipFree(partial);
    return rc;
}

// ------------------------------------------------------------------ engine
struct DevTensor {
    uint32_t type = 0;
    uint32_t nd = 0;
    uint64_t ne[4] = {1, 1, 1, 1};
    void *dev = nullptr;
    void *tdev = nullptr; // router weights [ROUTE_WIDTH][ROUTE_EXPERTS]: the transposed copy
    // router weights: max |w| (at upload), and at finalize their binary16 hi / lo
    // split of w * rscale (hi [E][dim] then lo), which the large calls' router reads
    float amax = 0.f, rscale = 1.f;
    void *rsplit = nullptr;
    size_t nbytes = 0;
    Q6T q6{};
    void *tiles_dev = nullptr; // prefill GEMM weights: the 32-row tile copy (at finalize)
    void *h16_dev = nullptr;   // and its binary16 fragment copy (tiles.h16; nullable)
    Q6Tiles tiles{};
};

struct lfm_engine {
    lfm_hparams hp{};
    int device = 0;
    uint32_t ctx = LFM_MAX_CTX;
    bool finalized = false;
    bool finalize_started = false; // device allocation of lfm_engine_finalize began
    hipStream_t stream = nullptr;
    Kernels *K = nullptr;
    std::unordered_map<std::string, DevTensor> tensors;
    std::string devname;

    DevState *st = nullptr;
    uint32_t *ids = nullptr, *out_tokens = nullptr;
    uint32_t *sel = nullptr;        // routing records, ROUTE_REC_WORDS per layer
    uint32_t last_route_layer = 0;  // the MoE layer whose record was enqueued last
    // prefill routing log (lfm_engine_set_route_log): per layer and prompt
    // position of the last multi-token call, ids[4], weights[4] and the router
    // logits [n_expert]; log_first[l] / log_n[l] give the token rows logged
    bool route_log = false;
    uint32_t *log_ids = nullptr;
    float *log_w = nullptr, *log_logits = nullptr;
    std::vector<uint32_t> log_first, log_n;
    std::vector<uint8_t> log_has_logits;
    float *x = nullptr, *y = nullptr, *qkv = nullptr, *sw = nullptr, *rlogits = nullptr,
          *logits = nullptr, *hpart = nullptr, *apart = nullptr;
    float *rpart = nullptr; // fused router expert partial sums [ROUTE_QUADS][ROUTE_PARTS] float4
    float *rss = nullptr;   // fused router x^2 partial sums [ROUTE_PARTS]
    float *xw = nullptr;    // fused router: the new residual times the FFN norm weight [dim]
    std::vector<uint16_t *> kc, vc;
    // attention layers: attn_q, attn_k and attn_v rows concatenated into one
    // Q6_K tensor (plane layout), so prefill projects q, k, v in one GEMM
    std::vector<Q6T> qkvw;
    std::vector<void *> qkvdev;
    std::vector<Q6Tiles> qkvt; // tile copies of qkvw (prefill)
    std::vector<void *> qkvtdev, qkvh16dev;
    std::vector<float *> conv;
    uint32_t head_grid = 1, nchunk = 1;
    float *rope = nullptr; // [ctx][32] (cos, sin)
    DevState *host_st = nullptr;    // pinned staging for state copies
    HostResult *host_res = nullptr; // pinned, device-mapped: forward calls' results
    HostResult *host_res_dev = nullptr; // its device address
    // batched prefill buffers (capacity: ctx tokens per call)
    struct {
        float *x = nullptr, *bcx = nullptr, *y = nullptr, *g = nullptr, *d = nullptr, *part = nullptr;
        float *cstate = nullptr; // the short conv's new state, until the next split copies it
        float *scale = nullptr, *logits = nullptr, *wsel = nullptr;
        uint16_t *hi = nullptr, *lo = nullptr;
        // small calls: the blocked activations' half-block scales (bscale, written by
        // the splits), and the SwiGLU output the gate/up GEMM stores split (hi2 / lo2
        // / bscale2, read by the down projection)
        float *bscale = nullptr, *bscale2 = nullptr;
        uint16_t *hi2 = nullptr, *lo2 = nullptr;
        uint32_t *sel = nullptr, *counts = nullptr, *tok = nullptr, *slot = nullptr, *pos = nullptr;
        // router partial sums left by the out projection's reduce (small calls), and
        // whether the current layer's were written
        float *rpart = nullptr, *rss = nullptr;
        bool router_ready = false;
        // small calls: the last MoE FFN's combine, left for the next layer's first
        // split to apply (comb_pending)
        ReduceCombineArgs comb{};
        bool comb_pending = false;
        // small calls: the conv state the next split moves from cstate into place
        float *state_pending = nullptr;
    } pf;
    uint32_t *host_ids = nullptr;   // pinned staging for prompt ids (ctx entries)

    // conv mixers of the captured step in one launch each (k_conv_mixer*): the
    // gated output's tagged entries, and whether the grid fits co-resident
    unsigned long long *flow = nullptr;
    bool fused_mixer = false;
    // set while capture() enqueues a step: only captured steps end with the
    // kernel that advances DevState::gen, which the fused kernels' tags need
    bool capturing = false;
    hipGraphExec_t g_layers = nullptr, g_decode = nullptr;
    hipEvent_t win_ev[2] = {nullptr, nullptr}; // lfm_decode_run's replay window
    uint64_t nodes_layers = 0, nodes_decode = 0;
    uint64_t dispatches = 0;
    bool stepwise_prefill = false; // true: prompts run as one decode step per token
};

static int engine_dev(lfm_engine *e)
{
    if (!e)
        return fail(LFM_EINVAL, "engine is null");
    HIPCHK(hipSetDevice(e->device));
    return LFM_OK;
}

static int validate_hparams(const lfm_hparams *hp)
{
    if (!hp)
        return fail(LFM_EINVAL, "hparams is null");
    if (hp->n_layers == 0 || hp->n_layers > LFM_MAX_LAYERS)
        return fail(LFM_EINVAL, "n_layers must be 1..%d", LFM_MAX_LAYERS);
    if (hp->dim == 0 || hp->dim % 256 || hp->dim > 2048)
        return fail(LFM_EINVAL, "dim must be a multiple of 256 up to 2048 (got %u)", hp->dim);
    if (hp->head_dim != 64 || hp->heads * hp->head_dim != hp->dim)
        return fail(LFM_EINVAL, "head_dim must be 64 and heads*head_dim == dim");
    for (uint32_t l = 0; l < hp->n_layers; ++l) {
        const uint32_t kv = hp->kv_heads[l];
        if (kv && (kv > 8 || hp->heads % kv || hp->heads / kv > 4))
            return fail(LFM_EINVAL, "layer %u: kv heads must divide heads, <= 8, heads/kv <= 4", l);
    }
    if (hp->vocab == 0)
        return fail(LFM_EINVAL, "vocab must be positive");
    if (hp->n_used == 0 || hp->n_used > 4 || hp->n_expert < hp->n_used || hp->n_expert > 64)
        return fail(LFM_EINVAL, "experts: need 1 <= n_used <= 4 and n_used <= n_expert <= 64");
    if (hp->expert_ff == 0 || hp->expert_ff % 256 || hp->expert_ff > 2048)
        return fail(LFM_EINVAL, "expert_ff must be a multiple of 256 up to 2048");
    if (hp->dense_lead > 0 && (hp->n_ff == 0 || hp->n_ff % 256 || hp->n_ff > 8192))
        return fail(LFM_EINVAL, "n_ff must be a multiple of 256 up to 8192");
    if (hp->conv_l_cache != 3)
        return fail(LFM_EINVAL, "shortconv l_cache must be 3");
    return LFM_OK;
}

extern "C" int lfm_engine_create(const lfm_hparams *hp, int device, lfm_engine **out)
{
    if (!out)
        return fail(LFM_EINVAL, "out is null");
    *out = nullptr;
    RC(validate_hparams(hp));
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(LFM_EDEVICE, "no HIP device available");
    if (device < 0 || device >= n)
        return fail(LFM_EINVAL, "device %d out of range (%d devices)", device, n);
    HIPCHK(hipSetDevice(device));
    lfm_engine *e = new lfm_engine();
    e->hp = *hp;
    e->device = device;
    // The marketing name can be blank (it is on some boards); then the name
    // falls back to the properties' name and finally to "AMD GPU <device>".
    char name[256] = {0};
    hipDeviceProp_t prop;
    memset(&prop, 0, sizeof(prop));
    if (hipDeviceGetName(name, sizeof(name) - 1, device) != hipSuccess)
        name[0] = 0;
    const bool have_prop = hipGetDeviceProperties(&prop, device) == hipSuccess;
    std::string nm = name;
    if (nm.empty() && have_prop)
        nm = prop.name;
    if (nm.empty())
        nm = "AMD GPU " + std::to_string(device);
    e->devname = have_prop && prop.gcnArchName[0] ? nm + " (" + prop.gcnArchName + ")" : nm;
    int rc = get_kernels(&e->K);
    if (rc == LFM_OK && hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess)
        rc = fail(LFM_EDEVICE, "hipStreamCreateWithFlags failed");
    if (rc != LFM_OK) {
        delete e;
        return rc;
    }
    *out = e;
    return LFM_OK;
}

extern "C" int lfm_engine_set_ctx(lfm_engine *e, uint32_t ctx)
{
    if (!e)
        return fail(LFM_EINVAL, "engine is null");
    if (e->finalized)
        return fail(LFM_ESTATE, "set_ctx must precede lfm_engine_finalize");
    if (ctx == 0 || ctx > LFM_MAX_CTX)
        return fail(LFM_ERANGE, "ctx must be 1..%d", LFM_MAX_CTX);
    e->ctx = ctx;
    return LFM_OK;
}

extern "C" int lfm_engine_hparams(const lfm_engine *e, lfm_hparams *out)
{
    if (!e || !out)
        return fail(LFM_EINVAL, "null argument");
    *out = e->hp;
    return LFM_OK;
}

int lfm_check_tensor(const char *name, uint32_t type, const uint64_t *ne, uint32_t nd,
                     size_t *want)
{
    if (!name || !ne || !want || nd == 0 || nd > 4)
        return fail(LFM_EINVAL, "tensor: bad arguments (name, shape, or 1..4 dimensions)");
    uint64_t n = 1;
    for (uint32_t i = 0; i < nd; ++i) {
        if (ne[i] == 0)
            return fail(LFM_EINVAL, "%s: dimension %u is zero", name, i);
        if (ne[i] > (1ull << 40) || n > (1ull << 40) / ne[i])
            return fail(LFM_EINVAL, "%s: %u-dimensional shape too large", name, nd);
        n *= ne[i];
    }
    if (type == LFM_GGML_TYPE_Q6_K) {
        if (ne[0] % 256)
            return fail(LFM_EINVAL, "%s: Q6_K row length %llu is not a multiple of 256", name,
                        (unsigned long long)ne[0]);
        *want = (size_t)(n / 256 * 210);
    } else if (type == LFM_GGML_TYPE_F32) {
        *want = (size_t)(n * 4);
    } else {
        return fail(LFM_EINVAL, "%s: unsupported ggml type %u (F32 and Q6_K only)", name, type);
    }
    return LFM_OK;
}

extern "C" int lfm_engine_upload_tensor(lfm_engine *e, const char *name, uint32_t type,
                                        const uint64_t *ne, uint32_t nd, const void *host,
                                        size_t nbytes)
{
    RC(engine_dev(e));
    if (e->finalized)
        return fail(LFM_ESTATE, "tensors must be uploaded before lfm_engine_finalize");
    if (!host)
        return fail(LFM_EINVAL, "upload_tensor: host pointer is null");
    size_t want = 0;
    RC(lfm_check_tensor(name, type, ne, nd, &want));
    DevTensor t;
    t.type = type;
    t.nd = nd;
    uint64_t n = 1;
    for (uint32_t i = 0; i < nd; ++i) {
        t.ne[i] = ne[i];
        n *= ne[i];
    }
    if (nbytes != want)
        return fail(LFM_EINVAL, "%s: %zu bytes given, %zu expected", name, nbytes, want);
    auto old = e->tensors.find(name);
    if (old != e->tensors.end()) {
        (void)hipFree(old->second.dev);
        if (old->second.tdev)
            (void)hipFree(old->second.tdev);
        if (old->second.tiles_dev)
            (void)hipFree(old->second.tiles_dev);
        if (old->second.rsplit)
            (void)hipFree(old->second.rsplit);
        e->tensors.erase(old);
    }
    // Router weights at the fused router's shape ([ROUTE_WIDTH inputs] x
    // [ROUTE_EXPERTS experts], expert-major as in the file) also get a
    // transposed copy [input][expert]: the output projection reads one input
    // row's 32 weights as one 128-byte line.
    const size_t nlen = strlen(name), slen = strlen("ffn_gate_inp.weight");
    if (type == LFM_GGML_TYPE_F32 && nd == 2 && nlen >= slen && strcmp(name + nlen - slen, "ffn_gate_inp.weight") == 0) {
        const float *src = (const float *)host;
        for (size_t i = 0; i < n; ++i)
            t.amax = std::max(t.amax, fabsf(src[i]));
    }
    if (type == LFM_GGML_TYPE_F32 && nd == 2 && ne[0] == ROUTE_WIDTH && ne[1] == ROUTE_EXPERTS &&
        nlen >= slen && strcmp(name + nlen - slen, "ffn_gate_inp.weight") == 0) {
        std::vector<float> tr((size_t)ROUTE_WIDTH * ROUTE_EXPERTS);
        const float *src = (const float *)host;
        for (uint32_t ex = 0; ex < ROUTE_EXPERTS; ++ex)
            for (uint32_t k = 0; k < ROUTE_WIDTH; ++k)
                tr[(size_t)k * ROUTE_EXPERTS + ex] = src[(size_t)ex * ROUTE_WIDTH + k];
        HIPCHK(hipMalloc(&t.tdev, tr.size() * 4));
        if (hipMemcpy(t.tdev, tr.data(), tr.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipFree(t.tdev);
            return fail(LFM_EDEVICE, "%s: transposed copy failed", name);
        }
    }
    if (hipMalloc(&t.dev, want) != hipSuccess) {
        if (t.tdev)
            (void)hipFree(t.tdev);
        return fail(LFM_EDEVICE, "%s: device allocation of %zu bytes failed", name, want);
    }
    t.nbytes = want;
    hipError_t ce;
    if (type == LFM_GGML_TYPE_Q6_K) {
        std::vector<uint8_t> packed(want);
        pack_blocks((const uint8_t *)host, n / 256, packed.data());
        ce = hipMemcpy(t.dev, packed.data(), want, hipMemcpyHostToDevice);
        t.q6 = q6view(t.dev, n / ne[0], ne[0]);
    } else {
        ce = hipMemcpy(t.dev, host, want, hipMemcpyHostToDevice);
    }
    if (ce != hipSuccess) {
        (void)hipFree(t.dev);
        if (t.tdev)
            (void)hipFree(t.tdev);
        return fail(LFM_EDEVICE, "%s: upload of %zu bytes failed: %s", name, want,
                    hipGetErrorString(ce));
    }
    e->tensors[name] = t;
    return LFM_OK;
}

static DevTensor *tensor(lfm_engine *e, const char *fmt, uint32_t l = 0)
{
    char nm[128];
    snprintf(nm, sizeof(nm), fmt, l);
    auto it = e->tensors.find(nm);
    return it == e->tensors.end() ? nullptr : &it->second;
}
static const float *f32(lfm_engine *e, const char *fmt, uint32_t l = 0)
{
    return (const float *)tensor(e, fmt, l)->dev;
}
static Q6T q6(lfm_engine *e, const char *fmt, uint32_t l = 0) { return tensor(e, fmt, l)->q6; }
// the prefill GEMMs' tile copy (made at finalize for every GEMM weight)
static Q6Tiles q6tiles(lfm_engine *e, const char *fmt, uint32_t l = 0) { return tensor(e, fmt, l)->tiles; }

// ------------------------------------------------------------------ step plan
static XSrc xsrc(const float *x, const float *norm, float eps)
{
    XSrc s;
    memset(&s, 0, sizeof(s));
    s.x = x;
    s.norm_w = norm;
    s.eps = eps;
    return s;
}

// The router of MoE layer l is fused into the output projection before it and
// the gate/up kernel (k_q6_matvec_route + k_gateup8f) at the model's shape:
// 32 experts, width ROUTE_WIDTH.
static bool fused_router(const lfm_engine *e, uint32_t l)
{
    const lfm_hparams &hp = e->hp;
    return l >= hp.dense_lead && hp.n_expert == ROUTE_EXPERTS && hp.dim == ROUTE_WIDTH;
}

// Output projection of layer l's mixer (y += W x); with the fused router it
// also leaves the router's partial sums.  `fuse` is set when the layer's FFN
// is enqueued right after (the decode step); the single-layer entry points
// run each half on its own and keep the separate router kernel.
static int launch_out_proj(lfm_engine *e, uint32_t l, MatvecArgs &m, bool fuse)
{
    if (!fuse || !fused_router(e, l))
        return launch_matvec(e->K, m, e->stream);
    if (m.w.rows != ROUTE_WIDTH || m.w.nb > 8 || m.mode != 1)
        return fail(LFM_EINTERNAL, "fused router: unexpected output projection shape");
    MatvecRouteArgs ra;
    ra.m = m;
    ra.rwt = (const float *)tensor(e, "blk.%u.ffn_gate_inp.weight", l)->tdev;
    if (!ra.rwt)
        return fail(LFM_EINTERNAL, "fused router: layer %u has no transposed router weights", l);
    ra.rnorm = f32(e, "blk.%u.ffn_norm.weight", l);
    ra.rpart = e->rpart;
    ra.rss = e->rss;
    ra.xw = e->xw;
    return launch_t(e->K->matvec_route, dim3(ROUTE_PARTS), 64 * ROUTE_ROWS, 0, e->stream, ra);
}

// Fused-router gate/up (k_gateup8f): 8-wave workgroups, 2 (rank, row) items per wave.
static int launch_gateup_fused(lfm_engine *e, const GateUpArgs &g)
{
    const uint32_t items = e->hp.n_used * e->hp.expert_ff;
    return launch_t(e->K->gateup_f, dim3((items + 15) / 16), 512, 0, e->stream, g);
}

// The conv mixer of a captured step in one launch (k_conv_mixer, or
// k_conv_mixer_r with the fused router's partial sums): dim / 8 workgroups of
// 8 waves, one channel and one output row per wave.
static int launch_conv_mixer(lfm_engine *e, uint32_t l, const ConvInprojArgs &in, const MatvecArgs &m)
{
    ConvMixerArgs a;
    memset(&a, 0, sizeof(a));
    a.in = in;
    a.out.m = m;
    a.flow = e->flow;
    a.phase = l;
    const bool route = fused_router(e, l);
    if (route) {
        if (m.w.rows != ROUTE_WIDTH || m.w.nb > 8 || m.mode != 1)
            return fail(LFM_EINTERNAL, "fused router: unexpected output projection shape");
        a.out.rwt = (const float *)tensor(e, "blk.%u.ffn_gate_inp.weight", l)->tdev;
        if (!a.out.rwt)
            return fail(LFM_EINTERNAL, "fused router: layer %u has no transposed router weights", l);
        a.out.rnorm = f32(e, "blk.%u.ffn_norm.weight", l);
        a.out.rpart = e->rpart;
        a.out.rss = e->rss;
        a.out.xw = e->xw;
    }
    if (in.dim % 8 || m.w.rows != in.dim || m.in_dim != in.dim)
        return fail(LFM_EINTERNAL, "conv mixer: unexpected shapes");
    RC(launch_t(route ? e->K->conv_mixer_r : e->K->conv_mixer, dim3(in.dim / 8), 512, 0, e->stream, a));
    e->dispatches += 1;
    return LFM_OK;
}

static int enq_mixer(lfm_engine *e, uint32_t l, bool embed, bool fuse)
{
    const lfm_hparams &hp = e->hp;
    const uint32_t dim = hp.dim, kv = hp.kv_heads[l];
    XSrc src = xsrc(e->x, f32(e, "blk.%u.attn_norm.weight", l), hp.eps);
    if (embed) {
        src.embed = 1;
        src.emb = q6(e, "token_embd.weight");
        src.x_out = e->x;
    }
    MatvecArgs m;
    memset(&m, 0, sizeof(m));
    m.src = xsrc(e->y, nullptr, 0.f);
    m.y = e->x;
    m.in_dim = dim;
    m.mode = 1;
    m.st = e->st;
    if (kv == 0) {
        ConvInprojArgs a;
        a.w = q6(e, "blk.%u.shortconv.in_proj.weight", l);
        a.src = src;
        a.conv_w = f32(e, "blk.%u.shortconv.conv.weight", l);
        a.state = e->conv[l];
        a.y = e->y;
        a.dim = dim;
        a.st = e->st;
        m.w = q6(e, "blk.%u.shortconv.out_proj.weight", l);
        if (fuse && !embed && e->fused_mixer && e->capturing)
            return launch_conv_mixer(e, l, a, m);
        RC(launch_mixer(e->K->conv, dim, e->stream, a));
        RC(launch_out_proj(e, l, m, fuse));
        e->dispatches += 2;
        return LFM_OK;
    }
    const uint32_t hdkv = 64 * kv;
    QkvArgs q;
    q.wq = q6(e, "blk.%u.attn_q.weight", l);
    q.wk = q6(e, "blk.%u.attn_k.weight", l);
    q.wv = q6(e, "blk.%u.attn_v.weight", l);
    q.src = src;
    q.qkv = e->qkv;
    q.dim = dim;
    q.hdkv = hdkv;
    q.st = e->st;
    RC(launch_mixer(e->K->qkv, dim + 2 * hdkv, e->stream, q));
    AttnArgs at;
    at.qkv = e->qkv;
    at.q_norm = f32(e, "blk.%u.attn_q_norm.weight", l);
    at.k_norm = f32(e, "blk.%u.attn_k_norm.weight", l);
    at.eps = hp.eps;
    at.rope = e->rope;
    at.scale = 1.0f / sqrtf((float)hp.head_dim);
    at.kcache = e->kc[l];
    at.vcache = e->vc[l];
    at.part = e->apart;
    at.ctx = e->ctx;
    at.heads = hp.heads;
    at.kv = kv;
    at.nchunk = e->nchunk;
    at.st = e->st;
    RC(launch(e->K->attn, dim3(e->nchunk, kv), 0, e->stream, at));
    AttnMergeArgs mg{e->apart, e->y, hp.heads, kv, e->nchunk, e->st};
    RC(launch(e->K->attn_merge, dim3(kv, hp.heads / kv), 0, e->stream, mg));
    m.w = q6(e, "blk.%u.attn_output.weight", l);
    RC(launch_out_proj(e, l, m, fuse));
    e->dispatches += 4;
    return LFM_OK;
}

static GateUpArgs moe_gateup_args(lfm_engine *e, uint32_t l)
{
    const lfm_hparams &hp = e->hp;
    GateUpArgs g;
    memset(&g, 0, sizeof(g));
    g.src = xsrc(e->x, f32(e, "blk.%u.ffn_norm.weight", l), hp.eps);
    g.sw = e->sw;
    g.st = e->st;
    g.route.logits = e->rlogits;
    g.route.bias = f32(e, "blk.%u.exp_probs_b.bias", l);
    g.route.n_expert = hp.n_expert;
    g.route.n_used = hp.n_used;
    g.route.sel_out = e->sel + (size_t)l * ROUTE_REC_WORDS;
    g.wg = q6(e, "blk.%u.ffn_gate_exps.weight", l);
    g.wu = q6(e, "blk.%u.ffn_up_exps.weight", l);
    g.ff = hp.expert_ff;
    return g;
}

static int enq_ffn(lfm_engine *e, uint32_t l, bool fuse)
{
    const lfm_hparams &hp = e->hp;
    const uint32_t dim = hp.dim;
    XSrc src = xsrc(e->x, f32(e, "blk.%u.ffn_norm.weight", l), hp.eps);
    GateUpArgs g;
    memset(&g, 0, sizeof(g));
    g.src = src;
    g.sw = e->sw;
    g.st = e->st;
    if (l < hp.dense_lead) {
        g.wg = q6(e, "blk.%u.ffn_gate.weight", l);
        g.wu = q6(e, "blk.%u.ffn_up.weight", l);
        g.ff = hp.n_ff;
        RC(launch_shape(e->K->gateup, hp.n_ff, e->stream, g));
        MatvecArgs m;
        memset(&m, 0, sizeof(m));
        m.w = q6(e, "blk.%u.ffn_down.weight", l);
        m.src = xsrc(e->sw, nullptr, 0.f);
        m.y = e->x;
        m.in_dim = hp.n_ff;
        m.mode = 1;
        m.st = e->st;
        RC(launch_matvec(e->K, m, e->stream));
        e->dispatches += 2;
        return LFM_OK;
    }
    const bool fused = fuse && fused_router(e, l);
    if (!fused) {
        RouterArgs r;
        r.src = src;
        r.w = f32(e, "blk.%u.ffn_gate_inp.weight", l);
        r.logits = e->rlogits;
        r.dim = dim;
        r.n_expert = hp.n_expert;
        r.st = e->st;
        RC(launch(e->K->router, dim3(hp.n_expert), 0, e->stream, r));
    }
    g = moe_gateup_args(e, l);
    if (fused) {
        g.route.logits = nullptr;
        g.route.rpart = e->rpart;
        g.route.rss = e->rss;
        g.route.xw = e->xw;
        RC(launch_gateup_fused(e, g));
    } else {
        RC(launch_shape(e->K->gateup, hp.n_used * hp.expert_ff, e->stream, g));
    }
    const Route route = g.route;
    MoeDownArgs d;
    d.wd = q6(e, "blk.%u.ffn_down_exps.weight", l);
    d.sw = e->sw;
    d.route = route;
    d.route.sel_out = g.route.sel_out; // the routing record stored by the gate/up kernel
    e->last_route_layer = l;
    d.x = e->x;
    d.dim = dim;
    d.ff = hp.expert_ff;
    d.st = e->st;
    if (!d.route.sel_out)
        return fail(LFM_EINTERNAL, "down projection launched without the routing buffer");
    RC(launch_t(e->K->moe_down, dim3((dim + 7) / 8), 1024, 0, e->stream, d));
    e->dispatches += fused ? 2 : 3;
    return LFM_OK;
}

// x: the residual to finish (the decode state's e->x, or a prefill's last row);
// host: nullable device address of pinned memory that also receives the result.
static int enq_head(lfm_engine *e, uint32_t advance, const float *x = nullptr, HostResult *host = nullptr)
{
    HeadArgs h;
    h.emb = q6(e, "token_embd.weight");
    h.src = xsrc(x ? x : e->x, f32(e, "token_embd_norm.weight"), e->hp.eps);
    h.logits = e->logits;
    h.partial = e->hpart;
    h.vocab = e->hp.vocab;
    h.st = e->st;
    RC(launch_t(e->K->head.fn(), dim3(e->head_grid), e->K->head.threads(), 0, e->stream, h));
    FinalArgs f{e->hpart, e->head_grid, e->out_tokens, advance, e->st, host};
    RC(launch(e->K->argmax_final, dim3(1), 0, e->stream, f));
    e->dispatches += 2;
    return LFM_OK;
}

static int enq_advance(lfm_engine *e)
{
    AdvanceArgs a{e->ids, e->st};
    RC(launch(e->K->advance, dim3(1), 0, e->stream, a));
    e->dispatches += 1;
    return LFM_OK;
}

static int enq_layers(lfm_engine *e)
{
    for (uint32_t l = 0; l < e->hp.n_layers; ++l) {
        RC(enq_mixer(e, l, l == 0, true));
        RC(enq_ffn(e, l, true));
    }
    return LFM_OK;
}

static int capture(lfm_engine *e, bool decode, hipGraphExec_t *exec, uint64_t *nodes)
{
    const uint64_t before = e->dispatches;
    hipGraph_t g = nullptr;
    HIPCHK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    e->capturing = true;
    int rc = enq_layers(e);
    if (rc == LFM_OK)
        rc = decode ? enq_head(e, 1) : enq_advance(e);
    e->capturing = false;
    hipError_t ce = hipStreamEndCapture(e->stream, &g);
    *nodes = e->dispatches - before;
    e->dispatches = before;
    if (rc != LFM_OK) {
        if (g)
            (void)hipGraphDestroy(g);
        return rc;
    }
    if (ce != hipSuccess)
        return fail(LFM_EDEVICE, "hipStreamEndCapture: %s", hipGetErrorString(ce));
    hipError_t ie = hipGraphInstantiate(exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ie != hipSuccess)
        return fail(LFM_EDEVICE, "hipGraphInstantiate: %s", hipGetErrorString(ie));
    return LFM_OK;
}

// The fused conv mixer (LFM_FUSED_MIXER=1 at finalize; off by default: on the
// MI355X its in-kernel handoff takes ~3.3 us after the last producer's store,
// more than the kernel boundary it replaces, and the step is 0.75 ms against
// 0.64 ms for the two-kernel chain).  Its workgroups wait for each other, so
// the whole grid (dim / 8 workgroups of 512 threads) must be resident at once:
// it is used only when the occupancy the runtime reports covers the grid.
static int check_fused_mixer(lfm_engine *e)
{
    e->fused_mixer = false;
    const char *env = getenv("LFM_FUSED_MIXER");
    if (!env || env[0] != '1')
        return LFM_OK;
    int cus = 0, per_cu = 0, per_cu_r = 0;
    HIPCHK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, e->device));
    HIPCHK(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, e->K->conv_mixer, 512, 0));
    HIPCHK(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_r, e->K->conv_mixer_r, 512, 0));
    const uint64_t grid = e->hp.dim / 8;
    e->fused_mixer = (uint64_t)std::min(per_cu, per_cu_r) * (uint64_t)cus >= grid;
    return LFM_OK;
}

extern "C" int lfm_engine_finalize(lfm_engine *e)
{
    RC(engine_dev(e));
    if (e->finalized)
        return fail(LFM_ESTATE, "engine already finalized");
    const lfm_hparams &hp = e->hp;
    // every tensor of the model must be present with the reference's shape
    const int count = lfm_model_tensor_count(&hp);
    for (int i = 0; i < count; ++i) {
        lfm_tensor_desc d;
        RC(lfm_model_tensor_desc(&hp, nullptr, i, &d));
        auto it = e->tensors.find(d.name);
        if (it == e->tensors.end())
            return fail(LFM_EINVAL, "missing tensor %s", d.name);
        const DevTensor &t = it->second;
        bool ok = t.type == d.ggml_type && t.nd == d.n_dims;
        for (uint32_t k = 0; ok && k < d.n_dims; ++k)
            ok = t.ne[k] == d.ne[k];
        if (!ok)
            return fail(LFM_EINVAL, "tensor %s has the wrong type or shape", d.name);
    }
    // From here on device buffers are allocated; a failure part-way leaves the
    // engine to be destroyed (a second attempt would allocate them again).
    if (e->finalize_started)
        return fail(LFM_ESTATE, "an earlier lfm_engine_finalize failed part-way; destroy the engine");
    e->finalize_started = true;
    const uint32_t dim = hp.dim;
    uint32_t max_hdkv = 0;
    for (uint32_t l = 0; l < hp.n_layers; ++l)
        max_hdkv = std::max(max_hdkv, 64 * hp.kv_heads[l]);
    e->nchunk = (e->ctx + 127) / 128;
    e->head_grid = e->K->head.grid(hp.vocab);
    {
        // NEOX RoPE angles as lfm.rs:251-256 computes them: tscale = theta^(-2/hd)
        // (powf), theta_p = pos * tscale^p with f32 square-and-multiply powi, then
        // sinf / cosf; tabulated once for every position of the context.
        const float tscale = powf(hp.rope_theta, -2.0f / (float)hp.head_dim);
        std::vector<float> tab((size_t)e->ctx * 64);
        for (uint32_t p = 0; p < 32; ++p) {
            float r = 1.0f, a = tscale;
            for (int b = (int)p;;) {
                if (b & 1)
                    r *= a;
                b /= 2;
                if (b == 0)
                    break;
                a *= a;
            }
            for (uint32_t pos = 0; pos < e->ctx; ++pos) {
                const float th = (float)pos * r;
                tab[(size_t)pos * 64 + 2 * p] = cosf(th);
                tab[(size_t)pos * 64 + 2 * p + 1] = sinf(th);
            }
        }
        HIPCHK(hipMalloc(&e->rope, tab.size() * 4));
        HIPCHK(hipMemcpy(e->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice));
    }
    const size_t swn = std::max<size_t>((size_t)hp.n_ff, (size_t)hp.n_used * hp.expert_ff);
    HIPCHK(hipHostMalloc((void **)&e->host_st, sizeof(DevState), hipHostMallocDefault));
    // forward calls' results, stored by the last kernel into host memory
    HIPCHK(hipHostMalloc((void **)&e->host_res, sizeof(HostResult), hipHostMallocCoherent | hipHostMallocMapped));
    HIPCHK(hipHostGetDevicePointer((void **)&e->host_res_dev, e->host_res, 0));
    HIPCHK(hipHostMalloc((void **)&e->host_ids, (size_t)e->ctx * 4, hipHostMallocDefault));
    HIPCHK(hipMalloc(&e->st, sizeof(DevState)));
    HIPCHK(hipMemset(e->st, 0, sizeof(DevState)));
    HIPCHK(hipMalloc(&e->ids, e->ctx * 4));
    HIPCHK(hipMalloc(&e->out_tokens, e->ctx * 4));
    HIPCHK(hipMalloc(&e->sel, (size_t)hp.n_layers * ROUTE_REC_WORDS * 4));
    HIPCHK(hipMemset(e->sel, 0, (size_t)hp.n_layers * ROUTE_REC_WORDS * 4));
    HIPCHK(hipMalloc(&e->x, dim * 4));
    HIPCHK(hipMalloc(&e->y, dim * 4));
    HIPCHK(hipMalloc(&e->qkv, (dim + 2 * max_hdkv) * 4));
    HIPCHK(hipMalloc(&e->sw, swn * 4));
    HIPCHK(hipMalloc(&e->rlogits, 64 * 4));
    HIPCHK(hipMalloc(&e->rpart, ROUTE_EXPERTS * ROUTE_PARTS * 4));
    HIPCHK(hipMalloc(&e->rss, ROUTE_PARTS * 4));
    HIPCHK(hipMalloc(&e->xw, ROUTE_WIDTH * 4));
    HIPCHK(hipMalloc(&e->flow, (size_t)dim * 8));
    HIPCHK(hipMemset(e->flow, 0, (size_t)dim * 8)); // tag 0 never matches
    RC(check_fused_mixer(e));
    HIPCHK(hipMemset(e->rpart, 0, ROUTE_EXPERTS * ROUTE_PARTS * 4));
    HIPCHK(hipMemset(e->rss, 0, ROUTE_PARTS * 4));
    HIPCHK(hipMemset(e->xw, 0, ROUTE_WIDTH * 4));
    HIPCHK(hipMalloc(&e->logits, (size_t)hp.vocab * 4));
    HIPCHK(hipMemset(e->logits, 0, (size_t)hp.vocab * 4));
    HIPCHK(hipMalloc(&e->hpart, e->head_grid * 2 * 4));
    HIPCHK(hipMalloc(&e->apart, (size_t)8 * e->nchunk * 4 * 66 * 4));
    e->qkvdev.assign(hp.n_layers, nullptr);
    e->qkvw.assign(hp.n_layers, Q6T{});
    for (uint32_t l = 0; l < hp.n_layers; ++l) {
        if (!hp.kv_heads[l])
            continue;
        const Q6T parts[3] = {q6(e, "blk.%u.attn_q.weight", l), q6(e, "blk.%u.attn_k.weight", l),
                              q6(e, "blk.%u.attn_v.weight", l)};
        const uint32_t rows = parts[0].rows + parts[1].rows + parts[2].rows, nb = parts[0].nb;
        const size_t nblk = (size_t)rows * nb;
        HIPCHK(hipMalloc(&e->qkvdev[l], nblk * 210));
        uint8_t *dst = (uint8_t *)e->qkvdev[l];
        // planes ql (128 B per block), qh (64), scales (16), d (2), each [rows][nb]
        const size_t pofs[4] = {0, 128, 192, 208}, psz[4] = {128, 64, 16, 2};
        for (int pl = 0; pl < 4; ++pl) {
            size_t at = nblk * pofs[pl];
            for (const Q6T &t : parts) {
                const size_t tb = (size_t)t.rows * t.nb;
                HIPCHK(hipMemcpy(dst + at, t.base + tb * pofs[pl], tb * psz[pl], hipMemcpyDeviceToDevice));
                at += tb * psz[pl];
            }
        }
        e->qkvw[l] = q6view(dst, rows, (uint64_t)nb * 256);
    }
    // The prefill GEMMs read their weights from 32-row tile copies (one contiguous
    // 1 KB / 512 B stretch per wave and load instead of 32 rows' pieces).  The
    // uploads and the qkv concatenation above are null-stream copies from pageable
    // memory, which may still be in flight when hipMemcpy returns and are not
    // ordered with the engine's non-blocking stream: finish them first.
    HIPCHK(hipDeviceSynchronize());
    e->qkvtdev.assign(hp.n_layers, nullptr);
    e->qkvh16dev.assign(hp.n_layers, nullptr);
    e->qkvt.assign(hp.n_layers, Q6Tiles{});
    for (uint32_t l = 0; l < hp.n_layers; ++l)
        if (hp.kv_heads[l]) {
            RC(make_tiles(e->K, e->stream, e->qkvw[l], e->qkvw[l].rows, &e->qkvtdev[l], &e->qkvt[l]));
            RC(make_h16(e->K, e->stream, &e->qkvt[l], &e->qkvh16dev[l]));
        }
    static const char *const gemm_weights[] = {"shortconv.in_proj.weight", "shortconv.out_proj.weight",
                                               "attn_output.weight",       "ffn_gate.weight",
                                               "ffn_up.weight",            "ffn_down.weight",
                                               "ffn_gate_exps.weight",     "ffn_up_exps.weight",
                                               "ffn_down_exps.weight"};
    for (auto &kv : e->tensors) {
        DevTensor &t = kv.second;
        const size_t n = kv.first.size();
        bool gemm = false;
        for (const char *suf : gemm_weights) {
            const size_t m = strlen(suf);
            gemm = gemm || (n > m && kv.first.compare(n - m, m, suf) == 0 && kv.first[n - m - 1] == '.');
        }
        if (gemm && t.type == LFM_GGML_TYPE_Q6_K && t.nd >= 2 && !t.tiles_dev) {
            RC(make_tiles(e->K, e->stream, t.q6, (uint32_t)t.ne[1], &t.tiles_dev, &t.tiles));
            // not for the experts' gate / up pair: its binary16 copy (2.4 times 193 MB
            // per layer) streams from HBM at every large call, where the Q6_K bytes
            // and their decode in registers measured faster (the other weights are
            // read by several token tiles through the caches)
            const bool pair_exps = ends_with(kv.first, "ffn_gate_exps.weight") || ends_with(kv.first, "ffn_up_exps.weight");
            if (!pair_exps)
                RC(make_h16(e->K, e->stream, &t.tiles, &t.h16_dev));
        }
        // router rows for the large calls' matrix-core router: w * 2^s in binary16
        // hi + lo, 2^s putting max |w| in [2^13, 2^14) so the lo halves stay normal
        const size_t rl = strlen("ffn_gate_inp.weight");
        if (t.type == LFM_GGML_TYPE_F32 && t.nd == 2 && !t.rsplit && n > rl &&
            kv.first.compare(n - rl, rl, "ffn_gate_inp.weight") == 0) {
            const uint64_t cnt = t.ne[0] * t.ne[1];
            int ex = 0;
            if (t.amax > 0.f && std::isfinite(t.amax))
                frexpf(t.amax, &ex);
            t.rscale = t.amax > 0.f && std::isfinite(t.amax) ? ldexpf(1.0f, 14 - ex) : 1.0f;
            HIPCHK(hipMalloc(&t.rsplit, cnt * 4));
            RouterSplitArgs ra{(const float *)t.dev, (uint16_t *)t.rsplit, (uint16_t *)t.rsplit + cnt, (uint32_t)cnt,
                               t.rscale};
            RC(launch_t(e->K->router_split, dim3((uint32_t)((cnt + 63) / 64)), 64, 0, e->stream, ra));
        }
    }
    HIPCHK(hipStreamSynchronize(e->stream));
    e->kc.assign(hp.n_layers, nullptr);
    e->vc.assign(hp.n_layers, nullptr);
    e->conv.assign(hp.n_layers, nullptr);
    for (uint32_t l = 0; l < hp.n_layers; ++l) {
        if (hp.kv_heads[l]) {
            const size_t n = (size_t)hp.kv_heads[l] * e->ctx * 64 * 2;
            HIPCHK(hipMalloc(&e->kc[l], n));
            HIPCHK(hipMalloc(&e->vc[l], n));
            HIPCHK(hipMemset(e->kc[l], 0, n));
            HIPCHK(hipMemset(e->vc[l], 0, n));
        } else {
            HIPCHK(hipMalloc(&e->conv[l], (size_t)dim * 2 * 4));
            HIPCHK(hipMemset(e->conv[l], 0, (size_t)dim * 2 * 4));
        }
    }
    {
        // batched prefill buffers, sized for a whole context in one call
        const size_t TC = e->ctx, E = hp.n_expert;
        const size_t wide = std::max<size_t>((size_t)hp.n_ff, 4 * (size_t)hp.expert_ff);
        // row-major hi / lo of a large call, or the token-blocked ones of a small call
        // (rows padded to 32; the grouped expert inputs reserve a padded list per expert)
        const size_t ts = (std::min<size_t>(TC, GEMM_TOKENS) + 31) / 32 * 32;
        const size_t kmax = std::max<size_t>({(size_t)dim, (size_t)hp.n_ff, (size_t)hp.expert_ff});
        const size_t hmax = std::max<size_t>({TC * dim, TC * hp.n_ff, TC * 4 * hp.expert_ff, ts * kmax,
                                              E * ts * std::max<size_t>(dim, hp.expert_ff)});
        const size_t bcxw = std::max<size_t>(3 * (size_t)dim, (size_t)dim + 2 * max_hdkv);
        HIPCHK(hipMalloc(&e->pf.x, TC * dim * 4));
        HIPCHK(hipMalloc(&e->pf.bcx, TC * bcxw * 4));
        HIPCHK(hipMalloc(&e->pf.y, TC * dim * 4));
        HIPCHK(hipMalloc(&e->pf.g, TC * wide * 4));
        HIPCHK(hipMalloc(&e->pf.d, TC * 4 * dim * 4));
        HIPCHK(hipMalloc(&e->pf.part, GEMM_PART_BYTES));
        if (hmax * 2 > 0x7fffffffull) // the GEMM kernels use 32-bit byte offsets into hi / lo
            return fail(LFM_ERANGE, "prefill activation copies of %zu bytes exceed 2 GiB", hmax * 2);
        HIPCHK(hipMalloc(&e->pf.hi, hmax * 2));
        HIPCHK(hipMalloc(&e->pf.lo, hmax * 2));
        HIPCHK(hipMalloc(&e->pf.scale, TC * 4 * 4));
        {
            // small calls' logical rows: a padded list per expert (grouped) or the call's
            const size_t lrows = std::max<size_t>(ts, E * ts), fmax = std::max<size_t>(hp.n_ff, hp.expert_ff);
            const size_t h2 = std::max<size_t>(E * ts * hp.expert_ff, ts * hp.n_ff);
            HIPCHK(hipMalloc(&e->pf.bscale, lrows * (kmax / 128) * 4));
            HIPCHK(hipMalloc(&e->pf.bscale2, lrows * (fmax / 128) * 4));
            HIPCHK(hipMalloc(&e->pf.hi2, h2 * 2));
            HIPCHK(hipMalloc(&e->pf.lo2, h2 * 2));
        }
        HIPCHK(hipMalloc(&e->pf.cstate, (size_t)dim * 2 * 4));
        const size_t tsmall = std::min<size_t>(TC, GEMM_TOKENS);
        HIPCHK(hipMalloc(&e->pf.rpart, tsmall * (dim / 256) * E * 4));
        HIPCHK(hipMalloc(&e->pf.rss, tsmall * (dim / 256) * 4));
        HIPCHK(hipMalloc(&e->pf.logits, TC * E * 4));
        HIPCHK(hipMalloc(&e->pf.wsel, TC * 4 * 4));
        HIPCHK(hipMalloc(&e->pf.sel, TC * 4 * 4));
        HIPCHK(hipMalloc(&e->pf.pos, TC * 4 * 4));
        HIPCHK(hipMalloc(&e->pf.counts, E * 4));
        HIPCHK(hipMalloc(&e->pf.tok, E * TC * 4));
        HIPCHK(hipMalloc(&e->pf.slot, E * TC * 4));
    }
    HIPCHK(hipDeviceSynchronize());
    RC(capture(e, false, &e->g_layers, &e->nodes_layers));
    RC(capture(e, true, &e->g_decode, &e->nodes_decode));
    for (hipEvent_t &ev : e->win_ev)
        HIPCHK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    e->finalized = true;
    return LFM_OK;
}

extern "C" void lfm_engine_destroy(lfm_engine *e)
{
    if (!e)
        return;
    (void)hipSetDevice(e->device);
    if (e->stream)
        (void)hipStreamSynchronize(e->stream);
    if (e->g_layers)
        (void)hipGraphExecDestroy(e->g_layers);
    if (e->g_decode)
        (void)hipGraphExecDestroy(e->g_decode);
    for (hipEvent_t ev : e->win_ev)
        if (ev)
            (void)hipEventDestroy(ev);
    for (auto &kv : e->tensors) {
        (void)hipFree(kv.second.dev);
        if (kv.second.tdev)
            (void)hipFree(kv.second.tdev);
        if (kv.second.tiles_dev)
            (void)hipFree(kv.second.tiles_dev);
        if (kv.second.h16_dev)
            (void)hipFree(kv.second.h16_dev);
        if (kv.second.rsplit)
            (void)hipFree(kv.second.rsplit);
    }
    for (void *p : e->qkvtdev)
        if (p)
            (void)hipFree(p);
    for (void *p : e->qkvh16dev)
        if (p)
            (void)hipFree(p);
    void *bufs[] = {e->st, e->ids, e->out_tokens, e->sel, e->log_ids, e->log_w, e->log_logits, e->flow, e->x, e->y, e->qkv, e->sw,
                    e->rlogits, e->rpart, e->rss, e->xw, e->logits, e->hpart, e->apart, e->rope,
                    e->pf.x, e->pf.bcx, e->pf.y, e->pf.g, e->pf.d, e->pf.part, e->pf.hi, e->pf.lo,
                    e->pf.bscale, e->pf.bscale2, e->pf.hi2, e->pf.lo2,
                    e->pf.scale, e->pf.logits, e->pf.wsel, e->pf.sel, e->pf.counts, e->pf.tok,
                    e->pf.slot, e->pf.pos, e->pf.cstate, e->pf.rpart, e->pf.rss};
    for (void *p : bufs)
        if (p)
            (void)hipFree(p);
    if (e->host_st)
        (void)hipHostFree(e->host_st);
    if (e->host_res)
        (void)hipHostFree(e->host_res);
    if (e->host_ids)
        (void)hipHostFree(e->host_ids);
    for (auto p : e->qkvdev)
        if (p)
            (void)hipFree(p);
    for (auto p : e->kc)
        if (p)
            (void)hipFree(p);
    for (auto p : e->vc)
        if (p)
            (void)hipFree(p);
    for (auto p : e->conv)
        if (p)
            (void)hipFree(p);
    if (e->stream)
        (void)hipStreamDestroy(e->stream);
    delete e;
}

// ------------------------------------------------------------------ batched prefill
// The multi-token forward (lfm.rs:290-694 with n > 1): every projection is a
// matrix-core GEMM over the T tokens of the call, the conv is parallel in t,
// attention is causal over the binary16 cache.  Leaves the last token's
// residual in row T - 1 of pf.x, which the head reads.
// RMSNorm (optional) + binary16 hi / lo split of `rows` activation rows for a
// GEMM of a T-token call: row-major for large calls, token-blocked for the
// small-call kernels (T <= GEMM_TOKENS), whose B reads expect that layout.
// grouped: the rows feed the expert GEMMs; spr = expert slots per row (4 for
// the token rows of the gate/up input, 1 for the slot rows of the down input).
// The split's arguments for `rows` rows of width K in a call of T tokens.
static SplitArgs split_args(lfm_engine *e, const float *x, const float *norm, uint32_t rows, uint32_t K,
                            uint32_t T, bool grouped = false, uint32_t spr = 1)
{
    SplitArgs a;
    memset(&a, 0, sizeof(a));
    a.x = x;
    a.norm_w = norm;
    a.eps = e->hp.eps;
    a.hi = e->pf.hi;
    a.lo = e->pf.lo;
    a.scale = e->pf.scale;
    a.bscale = e->pf.bscale;
    a.T = rows;
    a.K = K;
    a.mode = T > GEMM_TOKENS ? SPLIT_ROWMAJOR : grouped ? SPLIT_GROUPED : SPLIT_BLOCKED;
    if (a.mode == SPLIT_GROUPED) {
        a.sel = e->pf.sel;
        a.pos = e->pf.pos;
        a.spr = spr;
        a.n_used = e->hp.n_used;
        a.rpe = (T + 31) / 32 * 32;
    }
    return a;
}

// lists: (grouped, spr 4) form pos and the expert lists in the split itself;
// route (with lists): the split also routes each token from the router partials
// rg names.  A pending combine (small calls) of the rows of x is applied first.
static int pf_split(lfm_engine *e, const float *x, const float *norm, uint32_t rows, uint32_t K,
                    uint32_t T, bool grouped = false, uint32_t spr = 1, const float *copy_src = nullptr,
                    float *copy_dst = nullptr, uint32_t copy_n = 0, bool lists = false,
                    const RouteGroupArgs *route = nullptr)
{
    if (K == 0 || K % 256 || K > 8192) // k_split_rows keeps a row in registers
        return fail(LFM_EINVAL, "split: row width %u must be a multiple of 256 up to 8192", K);
    SplitArgs a = split_args(e, x, norm, rows, K, T, grouped, spr);
    a.copy_src = copy_src;
    a.copy_dst = copy_dst;
    a.copy_n = copy_n;
    if (e->pf.state_pending && !copy_src) { // a short conv's new state (small calls)
        a.copy_src = e->pf.cstate;
        a.copy_dst = e->pf.state_pending;
        a.copy_n = 2 * e->hp.dim;
        e->pf.state_pending = nullptr;
    }
    if (lists) {
        a.tok = e->pf.tok;
        a.slot = e->pf.slot;
        a.counts = e->pf.counts;
        a.list_stride = e->ctx;
        a.n_expert = e->hp.n_expert;
        if (route) {
            a.rpart = route->rpart;
            a.rss = route->rss;
            a.rbias = route->bias;
            a.sel_out = route->sel;
            a.wsel_out = route->wsel;
            a.logit_out = e->route_log ? e->pf.logits : nullptr;
            a.nparts = route->nparts;
        }
    }
    if (e->pf.comb_pending) {
        const ReduceCombineArgs &c = e->pf.comb;
        if (c.x != x || c.T != rows || c.dim != K)
            return fail(LFM_EINVAL, "split: a pending combine covers other rows");
        a.cpart = c.part;
        a.cwsel = c.wsel;
        a.cx = c.x;
        a.cksplit = c.ksplit;
        a.cn_used = c.n_used;
        e->pf.comb_pending = false;
    }
    RC(launch(a.cpart || a.tok ? e->K->split_rows_ext : e->K->split_rows, dim3(rows), 0, e->stream, a));
    e->dispatches += 1;
    return LFM_OK;
}

// act2 (small calls): the activations are the SwiGLU output that the pair GEMM
// stored split (pf.hi2 / lo2 / bscale2) instead of a split's.
static int pf_gemm(lfm_engine *e, const Q6Tiles &w, uint32_t T, float *c, uint32_t ldc, uint32_t col0,
                   uint32_t mode, uint32_t *deferred = nullptr, const RouterPart *router = nullptr,
                   bool *router_done = nullptr, bool act2 = false)
{
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.w = w;
    g.x_hi = act2 ? e->pf.hi2 : e->pf.hi;
    g.x_lo = act2 ? e->pf.lo2 : e->pf.lo;
    g.xscale = e->pf.scale;
    g.bscale = act2 ? e->pf.bscale2 : e->pf.bscale;
    g.ntok = T;
    g.zrows = w.rows;
    g.c = c;
    g.ldc = ldc;
    g.col0 = col0;
    g.mode = mode;
    return launch_gemm(e->K, e->stream, g, false, T, 1, T, 0, e->pf.part, GEMM_PART_BYTES / 4, &e->dispatches,
                       nullptr, nullptr, deferred, router, router_done);
}

// Gate and up projections of a SwiGLU FFN in one launch: c = silu(Wg x) * (Wu x)
// for `zrows` rows per weight (128 of each per workgroup).  Dense (tok null): the
// T tokens of the call; grouped: z = expert over the per-expert token lists, as
// pf_gemm_grouped.  Small calls store the output split for the down projection
// (pf.hi2 / lo2 / bscale2, its act2 input) instead of fp32 in c.
static int pf_gemm_swiglu(lfm_engine *e, const Q6Tiles &wg, const Q6Tiles &wu, uint32_t zrows, uint32_t T,
                          const uint32_t *tok, float *c, uint32_t ldc)
{
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.w = wg;
    g.w2 = wu;
    g.x_hi = e->pf.hi;
    g.x_lo = e->pf.lo;
    g.xscale = e->pf.scale;
    g.bscale = e->pf.bscale;
    g.ntok = T;
    g.zrows = zrows;
    g.c = c;
    g.ldc = ldc;
    if (T <= GEMM_TOKENS) {
        if (zrows % 128)
            return fail(LFM_EINTERNAL, "prefill: split SwiGLU output needs rows in 128s, not %u", zrows);
        g.y_hi = e->pf.hi2;
        g.y_lo = e->pf.lo2;
        g.y_bscale = e->pf.bscale2;
    }
    if (!tok)
        return launch_gemm(e->K, e->stream, g, true, T, 1, T, 0, e->pf.part, GEMM_PART_BYTES / 4, &e->dispatches);
    g.tok = tok;
    g.slot = e->pf.slot;
    g.counts = e->pf.counts;
    g.list_stride = e->ctx;
    g.rpz = (T + 31) / 32 * 32;
    return launch_gemm(e->K, e->stream, g, true, T, e->hp.n_expert, 4 * T, e->hp.n_used, e->pf.part,
                       GEMM_PART_BYTES / 4, &e->dispatches);
}

// Grouped expert GEMM: z = expert, rows zrows per expert, activation rows from
// `tok`, output rows `slot`, counts per expert on the device.
static int pf_gemm_grouped(lfm_engine *e, const Q6Tiles &w, uint32_t zrows, uint32_t T,
                           const uint32_t *tok, float *c, uint32_t ldc,
                           const CombinePrefillArgs *combine = nullptr, bool *combined = nullptr,
                           ReduceCombineArgs *defer_combine = nullptr, bool act2 = false)
{
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.w = w;
    g.x_hi = act2 ? e->pf.hi2 : e->pf.hi;
    g.x_lo = act2 ? e->pf.lo2 : e->pf.lo;
    g.xscale = e->pf.scale;
    g.bscale = act2 ? e->pf.bscale2 : e->pf.bscale;
    g.tok = tok;
    g.slot = e->pf.slot;
    g.counts = e->pf.counts;
    g.list_stride = e->ctx;
    g.rpz = (T + 31) / 32 * 32;
    g.zrows = zrows;
    g.c = c;
    g.ldc = ldc;
    return launch_gemm(e->K, e->stream, g, false, T, e->hp.n_expert, 4 * T, e->hp.n_used, e->pf.part,
                       GEMM_PART_BYTES / 4, &e->dispatches, combine, combined, nullptr, nullptr, nullptr,
                       defer_combine);
}

// The mixer's output projection, added to the residual.  Before a MoE FFN in a
// small call its reduce also leaves the router partial sums (e->pf.router_ready).
static int pf_out_proj(lfm_engine *e, uint32_t l, const Q6Tiles &w, uint32_t T)
{
    const lfm_hparams &hp = e->hp;
    e->pf.router_ready = false;
    if (l >= hp.dense_lead && T <= GEMM_TOKENS) {
        const RouterPart rp{f32(e, "blk.%u.ffn_norm.weight", l), f32(e, "blk.%u.ffn_gate_inp.weight", l), e->pf.rpart,
                            e->pf.rss, hp.n_expert, e->pf.counts};
        return pf_gemm(e, w, T, e->pf.x, hp.dim, 0, 1, nullptr, &rp, &e->pf.router_ready);
    }
    return pf_gemm(e, w, T, e->pf.x, hp.dim, 0, 1);
}

static int pf_mixer(lfm_engine *e, uint32_t l, uint32_t T, uint32_t start)
{
    const lfm_hparams &hp = e->hp;
    const uint32_t dim = hp.dim, kv = hp.kv_heads[l];
    RC(pf_split(e, e->pf.x, f32(e, "blk.%u.attn_norm.weight", l), T, dim, T));
    if (kv == 0) {
        // in_proj; with a K split the conv adds the slices itself (no reduce launch)
        uint32_t S = 1;
        RC(pf_gemm(e, q6tiles(e, "blk.%u.shortconv.in_proj.weight", l), T, e->pf.bcx, 3 * dim, 0, 0, &S));
        ConvPrefillArgs c{S > 1 ? e->pf.part : e->pf.bcx, f32(e, "blk.%u.shortconv.conv.weight", l), e->conv[l],
                          e->pf.cstate, e->pf.y, T, dim, S, nullptr, nullptr, nullptr};
        if (T <= GEMM_TOKENS) { // small calls: the conv stores y split for the out projection
            if (dim % 256)
                return fail(LFM_EINTERNAL, "prefill conv: width %u not a multiple of 256", dim);
            c.y_hi = e->pf.hi;
            c.y_lo = e->pf.lo;
            c.y_bscale = e->pf.bscale;
        }
        RC(launch(e->K->conv_prefill, dim3((dim + 255) / 256, T), 0, e->stream, c));
        if (T <= GEMM_TOKENS) // the FFN's split moves the new conv state into place
            e->pf.state_pending = e->conv[l];
        else // the split of y also moves the new conv state into place
            RC(pf_split(e, e->pf.y, nullptr, T, dim, T, false, 1, e->pf.cstate, e->conv[l], 2 * dim));
        RC(pf_out_proj(e, l, q6tiles(e, "blk.%u.shortconv.out_proj.weight", l), T));
        e->dispatches += 1;
        return LFM_OK;
    }
    const uint32_t hdkv = 64 * kv, w = dim + 2 * hdkv;
    // rows q | k | v = columns of bcx; with a K split the rope kernel adds the slices
    uint32_t S = 1;
    RC(pf_gemm(e, e->qkvt[l], T, e->pf.bcx, w, 0, 0, &S));
    RopeKvArgs r{e->pf.bcx, S > 1 ? e->pf.part : e->pf.bcx, f32(e, "blk.%u.attn_q_norm.weight", l),
                 f32(e, "blk.%u.attn_k_norm.weight", l), e->rope, hp.eps, e->kc[l], e->vc[l], T,
                 start, hp.heads, kv, e->ctx, S};
    RC(launch(e->K->rope_kv_prefill, dim3(T), 0, e->stream, r));
    AttnPrefillArgs at{e->pf.bcx, e->kc[l], e->vc[l], e->pf.y, 1.0f / sqrtf((float)hp.head_dim), T,
                       start, hp.heads, kv, e->ctx, nullptr, 0, 0};
    // Few query tiles (small calls, e.g. 64-token chunks late in the context): the
    // keys are split into ranges (about 256 workgroups, at least 4 blocks of 32
    // keys each) whose softmax states k_attn_merge_split combines.
    const uint32_t qtiles = (T + 31) / 32, nblk_max = (start + T - 1) / 32 + 1;
    uint32_t nsplit = 1, kb_per = 0;
    if (qtiles * kv < 128 && nblk_max >= 8) {
        kb_per = std::max<uint32_t>(4, (nblk_max * qtiles * kv + 255) / 256);
        nsplit = (nblk_max + kb_per - 1) / kb_per;
        if ((size_t)nsplit * T * hp.heads * 66 * 4 > GEMM_PART_BYTES)
            nsplit = 1, kb_per = 0;
    }
    if (nsplit > 1) {
        at.part = e->pf.part;
        at.kb_per = kb_per;
        RC(launch(e->K->attn_prefill, dim3(qtiles, kv, nsplit), 0, e->stream, at));
        AttnMergeSplitArgs mg{e->pf.part, e->pf.y, T, hp.heads, nsplit, nullptr, nullptr, nullptr};
        // small calls: the merge stores the output split for the output projection
        const bool direct = T <= GEMM_TOKENS && hp.heads % 4 == 0 && hp.heads * 64 == dim;
        if (direct) {
            mg.y_hi = e->pf.hi;
            mg.y_lo = e->pf.lo;
            mg.y_bscale = e->pf.bscale;
        }
        RC(launch(e->K->attn_merge_split, dim3(T, (hp.heads + 3) / 4), 0, e->stream, mg));
        e->dispatches += 1;
        if (!direct)
            RC(pf_split(e, e->pf.y, nullptr, T, dim, T));
    } else {
        at.paired = 1; // a long and a short query tile per workgroup
        RC(launch(e->K->attn_prefill, dim3((qtiles + 1) / 2, kv), 0, e->stream, at));
        RC(pf_split(e, e->pf.y, nullptr, T, dim, T));
    }
    RC(pf_out_proj(e, l, q6tiles(e, "blk.%u.attn_output.weight", l), T));
    e->dispatches += 2;
    return LFM_OK;
}

// FFN over T rows starting at x (the last layer runs only the last row).
// Prefill routing log: the routing of token rows first .. first + n - 1 at MoE
// layer l (and their router logits when the call computed them).
static int log_routes(lfm_engine *e, uint32_t l, uint32_t first, uint32_t n, bool logits)
{
    const uint32_t E = e->hp.n_expert;
    const size_t row = (size_t)l * e->ctx + first;
    HIPCHK(hipMemcpyAsync(e->log_ids + row * 4, e->pf.sel, (size_t)n * 16, hipMemcpyDeviceToDevice, e->stream));
    HIPCHK(hipMemcpyAsync(e->log_w + row * 4, e->pf.wsel, (size_t)n * 16, hipMemcpyDeviceToDevice, e->stream));
    if (logits)
        HIPCHK(hipMemcpyAsync(e->log_logits + row * E, e->pf.logits, (size_t)n * E * 4, hipMemcpyDeviceToDevice,
                              e->stream));
    e->log_first[l] = first;
    e->log_n[l] = n;
    e->log_has_logits[l] = logits ? 1 : 0;
    return LFM_OK;
}

// defer_ok: a split of the same rows follows (another layer), which may apply
// the MoE combine.
static int pf_ffn(lfm_engine *e, uint32_t l, float *x, uint32_t T, bool defer_ok)
{
    const lfm_hparams &hp = e->hp;
    const uint32_t dim = hp.dim;
    const float *norm = f32(e, "blk.%u.ffn_norm.weight", l);
    if (l < hp.dense_lead) {
        const uint32_t ff = hp.n_ff;
        RC(pf_split(e, x, norm, T, dim, T));
        RC(pf_gemm_swiglu(e, q6tiles(e, "blk.%u.ffn_gate.weight", l), q6tiles(e, "blk.%u.ffn_up.weight", l), ff, T,
                          nullptr, e->pf.g, ff));
        const bool act2 = T <= GEMM_TOKENS; // small calls: the pair stored its output split
        if (!act2)
            RC(pf_split(e, e->pf.g, nullptr, T, ff, T));
        RC(pf_gemm(e, q6tiles(e, "blk.%u.ffn_down.weight", l), T, x, dim, 0, 1, nullptr, nullptr, nullptr, act2));
        return LFM_OK;
    }
    const uint32_t eff = hp.expert_ff, E = hp.n_expert;
    RouterPrefillArgs ra{x, norm, f32(e, "blk.%u.ffn_gate_inp.weight", l), hp.eps, e->pf.logits, T,
                         dim, E};
    RouteGroupArgs rg{e->pf.logits, f32(e, "blk.%u.exp_probs_b.bias", l), e->pf.sel, e->pf.wsel,
                      e->pf.counts, e->pf.tok, e->pf.slot, T, E, hp.n_used, e->ctx, e->pf.pos,
                      nullptr, nullptr, 0, dim, hp.eps};
    if (e->pf.router_ready) { // the out projection's reduce left the router partials
        // x is token row `first` of the call's rows (the last layer runs only the last)
        const size_t first = (size_t)(x - e->pf.x) / dim, nb = dim / 256;
        rg.rpart = e->pf.rpart + first * nb * E;
        rg.rss = e->pf.rss + first * nb;
        rg.nparts = (uint32_t)nb;
    } else if (T <= GEMM_TOKENS) { // few tokens: one workgroup per (expert, token)
        RC(launch(e->K->router_small, dim3(E, T), 0, e->stream, ra));
        e->dispatches += 1;
    } else { // large calls: the FFN input's split first; the router reads its hi / lo
        RC(pf_split(e, x, norm, T, dim, T, true, 4));
        const DevTensor *rt = tensor(e, "blk.%u.ffn_gate_inp.weight", l);
        if (!rt || !rt->rsplit || rt->ne[0] != dim || rt->ne[1] != E)
            return fail(LFM_EINTERNAL, "prefill router: layer %u has no split router rows", l);
        const uint16_t *wh = (const uint16_t *)rt->rsplit;
        RouterMfmaArgs rm{e->pf.hi, e->pf.lo, e->pf.scale, wh, wh + (size_t)E * dim, 1.0f / rt->rscale,
                          e->pf.logits, T, dim, E};
        RC(launch(e->K->router_mfma, dim3((T + 31) / 32), 0, e->stream, rm));
        e->dispatches += 1;
    }
    // small calls: the split forms the expert lists itself (no k_route_group), and
    // with the out projection's router partials (and counts zeroed by its reduce) it
    // routes each token too (no k_route_topk)
    const bool small = T <= GEMM_TOKENS;
    const bool self_route = small && e->pf.router_ready;
    if (self_route && rg.nparts > 8) // dim <= 2048 (validate_hparams): at most 8 partials
        return fail(LFM_EINTERNAL, "prefill router: %u partial sums per token > 8", rg.nparts);
    if (!self_route) {
        RC(launch(e->K->route_topk, dim3((T + 3) / 4), 0, e->stream, rg));
        e->dispatches += 1;
    }
    if (!small) {
        RC(launch_t(e->K->route_group, dim3(E), 1024, 0, e->stream, rg));
        e->dispatches += 1;
    }
    if (small) // (large calls split before routing)
        RC(pf_split(e, x, norm, T, dim, T, true, 4, nullptr, nullptr, 0, true, self_route ? &rg : nullptr));
    if (e->route_log) // the call's routing is final here (ids, weights, logits)
        RC(log_routes(e, l, (uint32_t)((x - e->pf.x) / dim), T, true));
    RC(pf_gemm_swiglu(e, q6tiles(e, "blk.%u.ffn_gate_exps.weight", l), q6tiles(e, "blk.%u.ffn_up_exps.weight", l), eff,
                      T, e->pf.tok, e->pf.g, eff));
    if (!small) // (small calls: the pair stored its output split, per expert list)
        RC(pf_split(e, e->pf.g, nullptr, 4 * T, eff, T, true, 1)); // slots are token * 4 + rank
    CombinePrefillArgs cb{e->pf.d, e->pf.wsel, x, T, dim, hp.n_used};
    // small calls before another layer: the combine is left to the next layer's
    // first split (its rows are this call's, x = e->pf.x)
    const bool defer = small && defer_ok && x == e->pf.x;
    bool combined = false;
    RC(pf_gemm_grouped(e, q6tiles(e, "blk.%u.ffn_down_exps.weight", l), dim, T, e->pf.slot, e->pf.d, dim, &cb,
                       &combined, defer ? &e->pf.comb : nullptr, small));
    if (defer) {
        if (!combined) // one K slice: the down projection wrote d itself
            e->pf.comb = ReduceCombineArgs{e->pf.d, e->pf.wsel, x, 1, T, dim, hp.n_used};
        e->pf.comb_pending = true;
        return LFM_OK;
    }
    if (!combined)
        RC(launch(e->K->combine_prefill, dim3((dim + 1023) / 1024, T), 0, e->stream, cb)); // 4 k per thread
    e->dispatches += combined ? 0 : 1;
    return LFM_OK;
}

// Runs the layer stack for e->ids[0..T) at positions start.. and leaves the
// last token's residual in row T - 1 of pf.x.
// ids (nullable, T <= EMBED_INLINE_IDS): the call's ids, passed in the embedding
// launch's arguments, which also starts the decode state (no copies before it).
static int enq_prefill(lfm_engine *e, uint32_t T, uint32_t start, const uint32_t *ids = nullptr)
{
    const lfm_hparams &hp = e->hp;
    if (e->route_log)
        std::fill(e->log_n.begin(), e->log_n.end(), 0u);
    e->pf.comb_pending = false;
    e->pf.state_pending = nullptr;
    EmbedRowsArgs em;
    memset(&em, 0, sizeof(em));
    em.emb = q6(e, "token_embd.weight");
    em.ids = e->ids;
    em.x = e->pf.x;
    em.T = T;
    if (ids) {
        if (T > EMBED_INLINE_IDS)
            return fail(LFM_EINTERNAL, "prefill: %u inline ids > %u", T, EMBED_INLINE_IDS);
        em.ids = nullptr;
        memcpy(em.ids_inline, ids, (size_t)T * 4);
        em.st = e->st;
        em.start = start;
    }
    RC(launch(e->K->embed_rows, dim3((T + 3) / 4), 0, e->stream, em));
    e->dispatches += 1;
    for (uint32_t l = 0; l < hp.n_layers; ++l) {
        RC(pf_mixer(e, l, T, start));
        if (l + 1 < hp.n_layers)
            RC(pf_ffn(e, l, e->pf.x, T, true));
        else
            RC(pf_ffn(e, l, e->pf.x + (size_t)(T - 1) * hp.dim, 1, false));
    }
    if (e->pf.comb_pending) // cannot happen: the last layer combines itself
        return fail(LFM_ESTATE, "prefill: a combine was left pending");
    if (e->pf.state_pending) // cannot happen: every mixer is followed by its FFN's split
        return fail(LFM_ESTATE, "prefill: a conv state was left unmoved");
    return LFM_OK; // the last token's residual is row T - 1 of pf.x
}

// ------------------------------------------------------------------ forward
static int need_final(lfm_engine *e)
{
    RC(engine_dev(e));
    if (!e->finalized)
        return fail(LFM_ESTATE, "engine is not finalized");
    return LFM_OK;
}

// Writes the device-resident decode state.
static int set_state(lfm_engine *e, uint32_t tok, uint32_t pos, uint32_t n_ids, uint32_t eos)
{
    HIPCHK(hipStreamSynchronize(e->stream)); // the pinned staging block is reused
    DevState &h = *e->host_st;
    memset(&h, 0, sizeof(h));
    h.tok = tok;
    h.pos = pos;
    h.halt = 0;
    h.step = 0;
    h.eos = eos;
    h.cursor = 0;
    h.n_ids = n_ids;
    // everything but the step generation, which only the device advances
    HIPCHK(hipMemcpyAsync(e->st, &h, offsetof(DevState, gen), hipMemcpyHostToDevice, e->stream));
    return LFM_OK;
}

// Reads the device state back after the stream's work; a fused kernel's
// bounded handoff wait that timed out (the grid was not co-resident) fails the
// call that ran it.
static int read_state(lfm_engine *e, DevState *h)
{
    HIPCHK(hipMemcpyAsync(e->host_st, e->st, sizeof(DevState), hipMemcpyDeviceToHost, e->stream));
    HIPCHK(hipStreamSynchronize(e->stream));
    *h = *e->host_st;
    if (h->fault)
        return fail(LFM_EDEVICE, "a fused decode kernel's handoff wait timed out (workgroups not co-resident)");
    return LFM_OK;
}

static int check_ids(lfm_engine *e, const uint32_t *ids, uint32_t n, uint32_t start)
{
    if (!ids || n == 0)
        return fail(LFM_EINVAL, "token list must not be empty");
    if ((uint64_t)start + n > e->ctx)
        return fail(LFM_ERANGE, "forward context range: start %u + n %u > ctx %u", start, n, e->ctx);
    for (uint32_t j = 0; j < n; ++j)
        if (ids[j] >= e->hp.vocab)
            return fail(LFM_ERANGE, "token out of range: %u >= vocab %u", ids[j], e->hp.vocab);
    return LFM_OK;
}

static_assert(LFM_MAX_TOKEN_BATCH <= EMBED_INLINE_IDS, "forward_token batches fit the embedding launch's ids");

// Layers for every id (graph replays), then the head without feedback; the
// result also goes to the pinned e->host_res.
static int run_prompt(lfm_engine *e, const uint32_t *ids, uint32_t n, uint32_t start)
{
    RC(check_ids(e, ids, n, start));
    e->host_res->token = ~0u; // every earlier call has synchronized: no kernel writes it now
    const bool prefill = n >= 2 && !e->stepwise_prefill;
    if (prefill && n <= EMBED_INLINE_IDS) {
        // forward_token batches: the ids travel in the embedding launch's arguments,
        // which also starts the decode state (no copies ahead of the first kernel)
        RC(enq_prefill(e, n, start, ids));
    } else {
        RC(set_state(e, ids[0], start, n, 0xFFFFFFFFu)); // also waits for prior use of host_ids
        memcpy(e->host_ids, ids, (size_t)n * 4);
        HIPCHK(hipMemcpyAsync(e->ids, e->host_ids, (size_t)n * 4, hipMemcpyHostToDevice, e->stream));
        if (prefill) {
            RC(enq_prefill(e, n, start)); // matrix-core path
        } else {
            for (uint32_t j = 0; j < n; ++j) { // one captured decode step per token
                HIPCHK(hipGraphLaunch(e->g_layers, e->stream));
                e->dispatches += e->nodes_layers;
            }
        }
    }
    RC(enq_head(e, 0, prefill ? e->pf.x + (size_t)(n - 1) * e->hp.dim : e->x, e->host_res_dev));
    return LFM_OK;
}

extern "C" int lfm_forward_logits(lfm_engine *e, const uint32_t *ids, uint32_t n, uint32_t start,
                                  float *logits, size_t cap)
{
    RC(need_final(e));
    if (!logits || cap < e->hp.vocab)
        return fail(LFM_ERANGE, "logits buffer holds %zu < vocab %u floats", cap, e->hp.vocab);
    RC(run_prompt(e, ids, n, start));
    HIPCHK(hipMemcpyAsync(logits, e->logits, (size_t)e->hp.vocab * 4, hipMemcpyDeviceToHost,
                          e->stream));
    DevState h;
    return read_state(e, &h);
}

extern "C" int lfm_forward_token(lfm_engine *e, const uint32_t *ids, uint32_t n, uint32_t start,
                                 uint32_t *next, float *max_logit)
{
    RC(need_final(e));
    if (n == 0 || n > LFM_MAX_TOKEN_BATCH)
        return fail(LFM_EINVAL, "token batch must be 1..%d", LFM_MAX_TOKEN_BATCH);
    if (!next)
        return fail(LFM_EINVAL, "next is null");
    RC(run_prompt(e, ids, n, start));
    HIPCHK(hipStreamSynchronize(e->stream));
    const HostResult r = *e->host_res; // written by k_argmax_final (no copy back)
    if (r.token == ~0u) // not stored (a halted state): the state copy has the result
    {
        DevState h;
        RC(read_state(e, &h));
        *next = h.last_token;
        if (max_logit)
            *max_logit = h.last_value;
        return LFM_OK;
    }
    if (r.fault)
        return fail(LFM_EDEVICE, "a fused decode kernel's handoff wait timed out (workgroups not co-resident)");
    *next = r.token;
    if (max_logit)
        *max_logit = r.value;
    return LFM_OK;
}

extern "C" int lfm_decode_run(lfm_engine *e, uint32_t first, uint32_t start, uint32_t steps,
                              uint32_t eos, uint32_t *out_tokens, uint32_t *n_out)
{
    RC(need_final(e));
    if (!out_tokens || !n_out)
        return fail(LFM_EINVAL, "output pointers are null");
    *n_out = 0;
    if (steps == 0)
        return LFM_OK;
    if ((uint64_t)start + steps > e->ctx)
        return fail(LFM_ERANGE, "decode range: start %u + steps %u > ctx %u", start, steps, e->ctx);
    if (first >= e->hp.vocab)
        return fail(LFM_ERANGE, "token out of range: %u >= vocab %u", first, e->hp.vocab);
    RC(set_state(e, first, start, 0, eos));
    // At most 2 * DECODE_WINDOW replays are queued at once: before the replays
    // of window w the host waits for the event recorded after window w - 2.
    // The device stays fed (a whole window is still queued), and a caller or
    // tool that tracks every queued launch sees a bounded number of them.
    for (uint32_t s = 0; s < steps; ++s) {
        if (s % DECODE_WINDOW == 0 && s > 0) {
            hipEvent_t ev = e->win_ev[(s / DECODE_WINDOW) & 1];
            if (s >= 2 * DECODE_WINDOW)
                HIPCHK(hipEventSynchronize(ev));
            HIPCHK(hipEventRecord(ev, e->stream));
        }
        HIPCHK(hipGraphLaunch(e->g_decode, e->stream));
        e->dispatches += e->nodes_decode;
    }
    DevState h;
    RC(read_state(e, &h));
    const uint32_t n = std::min(h.step, steps);
    HIPCHK(hipMemcpy(out_tokens, e->out_tokens, (size_t)n * 4, hipMemcpyDeviceToHost));
    *n_out = n;
    return LFM_OK;
}

extern "C" int lfm_reset_session(lfm_engine *e)
{
    RC(need_final(e));
    for (uint32_t l = 0; l < e->hp.n_layers; ++l)
        if (e->conv[l])
            HIPCHK(hipMemsetAsync(e->conv[l], 0, (size_t)e->hp.dim * 2 * 4, e->stream));
    HIPCHK(hipStreamSynchronize(e->stream));
    return LFM_OK;
}

extern "C" int lfm_snapshot_bytes(const lfm_engine *e, uint32_t valid, size_t *nbytes)
{
    if (!e || !nbytes)
        return fail(LFM_EINVAL, "null argument");
    if (valid > e->ctx)
        return fail(LFM_ERANGE, "snapshot range: %u > ctx %u", valid, e->ctx);
    size_t total = 0;
    for (uint32_t l = 0; l < e->hp.n_layers; ++l)
        total += e->hp.kv_heads[l] ? 2 * (size_t)64 * e->hp.kv_heads[l] * valid * 4
                                   : (size_t)e->hp.dim * 2 * 4;
    *nbytes = total;
    return LFM_OK;
}

extern "C" int lfm_snapshot_cache(lfm_engine *e, uint32_t valid, uint8_t *buf, size_t cap,
                                  size_t *written)
{
    RC(need_final(e));
    size_t need;
    RC(lfm_snapshot_bytes(e, valid, &need));
    if (!buf || cap < need)
        return fail(LFM_ERANGE, "snapshot buffer holds %zu < %zu bytes", cap, need);
    HIPCHK(hipStreamSynchronize(e->stream));
    float *out = (float *)buf;
    size_t o = 0;
    std::vector<uint16_t> kh;
    for (uint32_t l = 0; l < e->hp.n_layers; ++l) {
        const uint32_t kv = e->hp.kv_heads[l];
        if (kv) {
            kh.resize((size_t)kv * e->ctx * 64);
            for (int which = 0; which < 2; ++which) {
                HIPCHK(hipMemcpy(kh.data(), which ? e->vc[l] : e->kc[l], kh.size() * 2,
                                 hipMemcpyDeviceToHost));
                for (uint32_t t = 0; t < valid; ++t)
                    for (uint32_t h = 0; h < kv; ++h)
                        for (uint32_t d = 0; d < 64; ++d)
                            out[o++] = lfm_f16_to_f32(kh[((size_t)h * e->ctx + t) * 64 + d]);
            }
        } else {
            HIPCHK(hipMemcpy(out + o, e->conv[l], (size_t)e->hp.dim * 2 * 4, hipMemcpyDeviceToHost));
            o += (size_t)e->hp.dim * 2;
        }
    }
    if (written)
        *written = need;
    return LFM_OK;
}

extern "C" int lfm_restore_session(lfm_engine *e, uint32_t valid, const uint8_t *buf, size_t len)
{
    RC(need_final(e));
    size_t need;
    RC(lfm_snapshot_bytes(e, valid, &need));
    if (!buf && len)
        return fail(LFM_EINVAL, "snapshot buffer is null");
    if (len < need)
        return fail(LFM_EINVAL, "truncated snapshot: %zu < %zu bytes", len, need);
    if (len > need)
        return fail(LFM_EINVAL, "extra snapshot data: %zu > %zu bytes", len, need);
    HIPCHK(hipStreamSynchronize(e->stream));
    const float *in = (const float *)buf;
    size_t o = 0;
    std::vector<uint16_t> kh;
    for (uint32_t l = 0; l < e->hp.n_layers; ++l) {
        const uint32_t kv = e->hp.kv_heads[l];
        if (kv) {
            kh.resize((size_t)kv * e->ctx * 64);
            for (int which = 0; which < 2; ++which) {
                uint16_t *dst = which ? e->vc[l] : e->kc[l];
                HIPCHK(hipMemcpyAsync(kh.data(), dst, kh.size() * 2, hipMemcpyDeviceToHost, e->stream));
                HIPCHK(hipStreamSynchronize(e->stream));
                for (uint32_t t = 0; t < valid; ++t)
                    for (uint32_t h = 0; h < kv; ++h)
                        for (uint32_t d = 0; d < 64; ++d)
                            kh[((size_t)h * e->ctx + t) * 64 + d] = lfm_f32_to_f16(in[o++]);
                HIPCHK(hipMemcpyAsync(dst, kh.data(), kh.size() * 2, hipMemcpyHostToDevice, e->stream));
                HIPCHK(hipStreamSynchronize(e->stream));
            }
        } else {
            HIPCHK(hipMemcpyAsync(e->conv[l], in + o, (size_t)e->hp.dim * 2 * 4, hipMemcpyHostToDevice,
                                  e->stream));
            HIPCHK(hipStreamSynchronize(e->stream));
            o += (size_t)e->hp.dim * 2;
        }
    }
    // (every copy above ran on the engine stream and was waited for before its
    // host buffer was reused: later engine work and the caller see the state)
    return LFM_OK;
}

extern "C" int lfm_snapshot_logits(lfm_engine *e, float *out, size_t cap)
{
    RC(need_final(e));
    if (!out || cap < e->hp.vocab)
        return fail(LFM_ERANGE, "logits buffer holds %zu < vocab %u floats", cap, e->hp.vocab);
    HIPCHK(hipStreamSynchronize(e->stream));
    HIPCHK(hipMemcpy(out, e->logits, (size_t)e->hp.vocab * 4, hipMemcpyDeviceToHost));
    return LFM_OK;
}

extern "C" uint64_t lfm_dispatch_count(const lfm_engine *e) { return e ? e->dispatches : 0; }

extern "C" int lfm_engine_h16_bytes(const lfm_engine *e, uint64_t *bytes)
{
    if (!e || !bytes)
        return fail(LFM_EINVAL, "lfm_engine_h16_bytes: null argument");
    uint64_t n = 0;
    for (const auto &kv : e->tensors)
        if (kv.second.h16_dev)
            n += (uint64_t)kv.second.tiles.tiles * kv.second.tiles.nb * TILE_H16;
    for (size_t l = 0; l < e->qkvh16dev.size(); ++l)
        if (e->qkvh16dev[l])
            n += (uint64_t)e->qkvt[l].tiles * e->qkvt[l].nb * TILE_H16;
    *bytes = n;
    return LFM_OK;
}

extern "C" int lfm_engine_set_prefill_mode(lfm_engine *e, int stepwise)
{
    if (!e)
        return fail(LFM_EINVAL, "engine is null");
    e->stepwise_prefill = stepwise != 0;
    return LFM_OK;
}

extern "C" int lfm_device_name(const lfm_engine *e, char *buf, size_t cap)
{
    if (!e || !buf || cap == 0)
        return fail(LFM_EINVAL, "null argument");
    snprintf(buf, cap, "%s", e->devname.c_str());
    return LFM_OK;
}

// ------------------------------------------------------------------ kernel timing
// Average duration of the routed gate/up kernel (the largest share of a decode
// step): one graph of `reps` rounds over every MoE layer's weights (their 4
// routed experts, > 256 MB in total, so the Infinity Cache cannot hold them),
// timed with HIP events on the engine stream.  The kernel is the one the
// decode step runs (with the fused router, k_gateup8f over the router partial
// sums of the last step; else k_gateup4 over the last router logits).
extern "C" int lfm_engine_time_moe_gateup(lfm_engine *e, uint32_t reps, float *us_per_launch,
                                          uint64_t *bytes_per_launch)
{
    RC(need_final(e));
    const lfm_hparams &hp = e->hp;
    if (!us_per_launch || !bytes_per_launch || reps == 0)
        return fail(LFM_EINVAL, "bad arguments");
    uint32_t nmoe = 0;
    for (uint32_t l = hp.dense_lead; l < hp.n_layers; ++l)
        ++nmoe;
    if (nmoe == 0)
        return fail(LFM_ESTATE, "model has no MoE layer");
    RC(set_state(e, 0, 0, 0, 0xFFFFFFFFu));
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    HIPCHK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    int rc = LFM_OK;
    const bool fused = fused_router(e, hp.dense_lead);
    for (uint32_t r = 0; r < reps && rc == LFM_OK; ++r)
        for (uint32_t l = hp.dense_lead; l < hp.n_layers && rc == LFM_OK; ++l) {
            GateUpArgs a = moe_gateup_args(e, l);
            if (fused) {
                a.route.logits = nullptr;
                a.route.rpart = e->rpart;
                a.route.rss = e->rss;
                a.route.xw = e->xw;
                rc = launch_gateup_fused(e, a);
            } else {
                rc = launch_shape(e->K->gateup, hp.n_used * hp.expert_ff, e->stream, a);
            }
        }
    hipError_t ce = hipStreamEndCapture(e->stream, &g);
    if (rc != LFM_OK || ce != hipSuccess) {
        if (g)
            (void)hipGraphDestroy(g);
        return rc != LFM_OK ? rc : fail(LFM_EDEVICE, "capture: %s", hipGetErrorString(ce));
    }
    hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ie != hipSuccess)
        return fail(LFM_EDEVICE, "hipGraphInstantiate: %s", hipGetErrorString(ie));
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    HIPCHK(hipGraphLaunch(ge, e->stream)); // warm
    HIPCHK(hipEventRecord(e0, e->stream));
    HIPCHK(hipGraphLaunch(ge, e->stream));
    HIPCHK(hipEventRecord(e1, e->stream));
    HIPCHK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIPCHK(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipGraphExecDestroy(ge);
    e->dispatches += 2ull * reps * nmoe;
    *us_per_launch = ms * 1e3f / (float)(reps * nmoe);
    // weights + input (x and the norm weight, or the fused router's x * w) +
    // router inputs (partial sums, or logits) and bias + output
    const uint64_t wbytes = 2ull * hp.n_used * hp.expert_ff * (hp.dim / 256) * 210;
    const uint64_t rbytes = fused ? (uint64_t)(ROUTE_EXPERTS + 1) * ROUTE_PARTS * 4 : hp.n_expert * 4ull;
    // ... and the layer's routing record (ids and weights, logits and scores)
    *bytes_per_launch = wbytes + (fused ? 1ull : 2ull) * hp.dim * 4 + rbytes + hp.n_expert * 4ull +
                        (uint64_t)hp.n_used * hp.expert_ff * 4 + (16ull + 2ull * hp.n_expert) * 4;
    return LFM_OK;
}

// Average duration of the final-norm + tied-head kernel (k_head*, the largest
// single matvec of a step: vocab x dim Q6_K) over one graph of `reps` rounds
// that rotate `ncopies` copies of the embedding planes (ncopies x 110 MB at the
// model's shape, beyond the 256 MB Infinity Cache from 3 copies on).
extern "C" int lfm_engine_time_head(lfm_engine *e, uint32_t ncopies, uint32_t reps,
                                    float *us_per_launch, uint64_t *bytes_per_launch)
{
    RC(need_final(e));
    if (!us_per_launch || !bytes_per_launch || reps == 0 || ncopies == 0 || ncopies > 8)
        return fail(LFM_EINVAL, "bad arguments");
    const Q6T emb = q6(e, "token_embd.weight");
    const size_t nbytes = (size_t)emb.rows * emb.nb * 210;
    std::vector<uint8_t *> copies(ncopies, nullptr);
    copies[0] = const_cast<uint8_t *>(emb.base);
    int rc = LFM_OK;
    for (uint32_t i = 1; i < ncopies && rc == LFM_OK; ++i) {
        if (hipMalloc(&copies[i], nbytes) != hipSuccess ||
            hipMemcpyAsync(copies[i], emb.base, nbytes, hipMemcpyDeviceToDevice, e->stream) != hipSuccess)
            rc = fail(LFM_EDEVICE, "head copies: %zu bytes", nbytes);
    }
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    float ms = 0.f;
    if (rc == LFM_OK) {
        rc = set_state(e, 0, 0, 0, 0xFFFFFFFFu);
        if (rc == LFM_OK && hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
            rc = fail(LFM_EDEVICE, "capture begin");
        if (rc == LFM_OK) {
            for (uint32_t r = 0; r < reps && rc == LFM_OK; ++r)
                for (uint32_t i = 0; i < ncopies && rc == LFM_OK; ++i) {
                    HeadArgs h;
                    h.emb = emb;
                    h.emb.base = copies[i];
                    h.src = xsrc(e->x, f32(e, "token_embd_norm.weight"), e->hp.eps);
                    h.logits = e->logits;
                    h.partial = e->hpart;
                    h.vocab = e->hp.vocab;
                    h.st = e->st;
                    rc = launch_t(e->K->head.fn(), dim3(e->head_grid), e->K->head.threads(), 0,
                                  e->stream, h);
                }
            hipError_t ce = hipStreamEndCapture(e->stream, &g);
            if (rc == LFM_OK && ce != hipSuccess)
                rc = fail(LFM_EDEVICE, "capture: %s", hipGetErrorString(ce));
        }
        if (rc == LFM_OK && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess)
            rc = fail(LFM_EDEVICE, "hipGraphInstantiate");
        if (g)
            (void)hipGraphDestroy(g);
        if (rc == LFM_OK) {
            hipEvent_t e0 = nullptr, e1 = nullptr;
            if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess ||
                hipGraphLaunch(ge, e->stream) != hipSuccess || hipEventRecord(e0, e->stream) != hipSuccess ||
                hipGraphLaunch(ge, e->stream) != hipSuccess || hipEventRecord(e1, e->stream) != hipSuccess ||
                hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
                rc = fail(LFM_EDEVICE, "head timing");
            if (e0)
                (void)hipEventDestroy(e0);
            if (e1)
                (void)hipEventDestroy(e1);
        }
        if (ge)
            (void)hipGraphExecDestroy(ge);
    }
    (void)hipStreamSynchronize(e->stream);
    for (uint32_t i = 1; i < ncopies; ++i)
        if (copies[i])
            (void)hipFree(copies[i]);
    RC(rc);
    e->dispatches += 2ull * reps * ncopies;
    *us_per_launch = ms * 1e3f / (float)(reps * ncopies);
    // weights + input vector + norm weight + logits + partials
    *bytes_per_launch = nbytes + 2ull * e->hp.dim * 4 + (uint64_t)e->hp.vocab * 4 + e->head_grid * 8ull;
    return LFM_OK;
}

// ------------------------------------------------------------------ layer entry points
static int run_layer_part(lfm_engine *e, uint32_t layer, float *x, uint32_t pos, bool mixer)
{
    RC(need_final(e));
    if (!x)
        return fail(LFM_EINVAL, "x is null");
    if (layer >= e->hp.n_layers)
        return fail(LFM_ERANGE, "layer %u >= %u", layer, e->hp.n_layers);
    if (pos >= e->ctx)
        return fail(LFM_ERANGE, "position %u >= ctx %u", pos, e->ctx);
    HIPCHK(hipMemcpyAsync(e->x, x, (size_t)e->hp.dim * 4, hipMemcpyHostToDevice, e->stream));
    RC(set_state(e, 0, pos, 0, 0xFFFFFFFFu));
    RC(mixer ? enq_mixer(e, layer, false, false) : enq_ffn(e, layer, false));
    HIPCHK(hipMemcpyAsync(x, e->x, (size_t)e->hp.dim * 4, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(hipStreamSynchronize(e->stream));
    return LFM_OK;
}

extern "C" int lfm_engine_run_mixer(lfm_engine *e, uint32_t layer, float *x, uint32_t pos)
{
    return run_layer_part(e, layer, x, pos, true);
}

extern "C" int lfm_engine_run_ffn(lfm_engine *e, uint32_t layer, float *x)
{
    return run_layer_part(e, layer, x, 0, false);
}

// One whole layer as the decode step runs it: the mixer, then the FFN enqueued
// right after with the router fused into the mixer's output projection (when
// the shape has the fused router), so the routing comes from the same kernels
// and the same partial sums as in the captured step.  x_mid (optional)
// receives the residual between the halves: the FFN's input.
extern "C" int lfm_engine_run_layer(lfm_engine *e, uint32_t layer, float *x, uint32_t pos,
                                    float *x_mid)
{
    RC(need_final(e));
    if (!x)
        return fail(LFM_EINVAL, "x is null");
    if (layer >= e->hp.n_layers)
        return fail(LFM_ERANGE, "layer %u >= %u", layer, e->hp.n_layers);
    if (pos >= e->ctx)
        return fail(LFM_ERANGE, "position %u >= ctx %u", pos, e->ctx);
    const size_t nb = (size_t)e->hp.dim * 4;
    HIPCHK(hipMemcpyAsync(e->x, x, nb, hipMemcpyHostToDevice, e->stream));
    RC(set_state(e, 0, pos, 0, 0xFFFFFFFFu));
    RC(enq_mixer(e, layer, false, true));
    if (x_mid)
        HIPCHK(hipMemcpyAsync(x_mid, e->x, nb, hipMemcpyDeviceToHost, e->stream));
    RC(enq_ffn(e, layer, true));
    HIPCHK(hipMemcpyAsync(x, e->x, nb, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(hipStreamSynchronize(e->stream));
    return LFM_OK;
}

// Whether MoE layer `layer` routes through the fused router in the decode step.
extern "C" int lfm_engine_fused_router(const lfm_engine *e, uint32_t layer, int *fused)
{
    if (!e || !fused)
        return fail(LFM_EINVAL, "null argument");
    if (layer >= e->hp.n_layers)
        return fail(LFM_ERANGE, "layer %u >= %u", layer, e->hp.n_layers);
    *fused = fused_router(e, layer) ? 1 : 0;
    return LFM_OK;
}

extern "C" int lfm_engine_last_route(lfm_engine *e, uint32_t *ids, float *w, uint32_t cap)
{
    RC(need_final(e));
    if (!ids || !w || cap < e->hp.n_used)
        return fail(LFM_ERANGE, "route buffers hold %u < %u entries", cap, e->hp.n_used);
    uint32_t h[16];
    HIPCHK(hipStreamSynchronize(e->stream));
    HIPCHK(hipMemcpy(h, e->sel + (size_t)e->last_route_layer * ROUTE_REC_WORDS, sizeof(h),
                     hipMemcpyDeviceToHost));
    for (uint32_t r = 0; r < e->hp.n_used; ++r) {
        ids[r] = h[r];
        memcpy(&w[r], &h[8 + r], 4);
    }
    return LFM_OK;
}

// The decode step's routing records, one per layer (zero for dense layers and
// layers not run since finalize).
extern "C" int lfm_engine_route_records(lfm_engine *e, uint32_t *words, size_t cap_words)
{
    RC(need_final(e));
    const size_t n = (size_t)e->hp.n_layers * ROUTE_REC_WORDS;
    if (!words || cap_words < n)
        return fail(LFM_ERANGE, "route record buffer holds %zu < %zu words", cap_words, n);
    HIPCHK(hipStreamSynchronize(e->stream));
    HIPCHK(hipMemcpy(words, e->sel, n * 4, hipMemcpyDeviceToHost));
    return LFM_OK;
}

extern "C" int lfm_engine_set_route_log(lfm_engine *e, int on)
{
    RC(need_final(e));
    if (on && !e->log_ids) { // all three buffers or none
        const size_t rows = (size_t)e->hp.n_layers * e->ctx;
        uint32_t *ids = nullptr;
        float *w = nullptr, *lg = nullptr;
        if (hipMalloc(&ids, rows * 16) != hipSuccess || hipMalloc(&w, rows * 16) != hipSuccess ||
            hipMalloc(&lg, rows * e->hp.n_expert * 4) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipFree(ids);
            (void)hipFree(w);
            (void)hipFree(lg);
            return fail(LFM_EDEVICE, "routing log: device allocation failed");
        }
        e->log_ids = ids;
        e->log_w = w;
        e->log_logits = lg;
        e->log_first.assign(e->hp.n_layers, 0u);
        e->log_n.assign(e->hp.n_layers, 0u);
        e->log_has_logits.assign(e->hp.n_layers, 0);
    }
    e->route_log = on != 0;
    return LFM_OK;
}

extern "C" int lfm_engine_prefill_routes(lfm_engine *e, uint32_t layer, uint32_t *first, uint32_t *n,
                                         int *has_logits, uint32_t *ids, float *w, float *logits,
                                         size_t cap_rows)
{
    RC(need_final(e));
    if (!e->log_ids)
        return fail(LFM_ESTATE, "routing log is off (lfm_engine_set_route_log)");
    if (layer >= e->hp.n_layers)
        return fail(LFM_ERANGE, "layer %u >= %u", layer, e->hp.n_layers);
    if (!first || !n || !has_logits || !ids || !w)
        return fail(LFM_EINVAL, "null argument");
    const uint32_t cnt = e->log_n[layer];
    if (cap_rows < cnt)
        return fail(LFM_ERANGE, "buffers hold %zu < %u rows", cap_rows, cnt);
    *first = e->log_first[layer];
    *n = cnt;
    *has_logits = e->log_has_logits[layer];
    HIPCHK(hipStreamSynchronize(e->stream));
    const size_t row = (size_t)layer * e->ctx + *first;
    if (cnt) {
        HIPCHK(hipMemcpy(ids, e->log_ids + row * 4, (size_t)cnt * 16, hipMemcpyDeviceToHost));
        HIPCHK(hipMemcpy(w, e->log_w + row * 4, (size_t)cnt * 16, hipMemcpyDeviceToHost));
        if (*has_logits && logits)
            HIPCHK(hipMemcpy(logits, e->log_logits + row * e->hp.n_expert, (size_t)cnt * e->hp.n_expert * 4,
                             hipMemcpyDeviceToHost));
    }
    return LFM_OK;
}

// ------------------------------------------------------------------ synthetic model
extern "C" int lfm_engine_load_synthetic(lfm_engine *e, const lfm_synth_opts *o, int threads)
{
    RC(engine_dev(e));
    const int count = lfm_model_tensor_count(&e->hp);
    if (count < 0)
        return fail(LFM_EINVAL, "bad hparams");
    std::vector<uint8_t> buf;
    for (int i = 0; i < count; ++i) {
        lfm_tensor_desc d;
        RC(lfm_model_tensor_desc(&e->hp, o, i, &d));
        const size_t nb = lfm_tensor_nbytes(&d);
        buf.resize(nb);
        RC(lfm_synth_tensor(o, &d, buf.data(), nb, threads));
        RC(lfm_engine_upload_tensor(e, d.name, d.ggml_type, d.ne, d.n_dims, buf.data(), nb));
    }
    return LFM_OK;
}
