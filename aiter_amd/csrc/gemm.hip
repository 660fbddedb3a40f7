// Host launchers and C-ABI entry points of the scaled-GEMM family.
//
// Every kernel instance has a stable name and integer id (the `kernelName` /
// `kernelId` the tuned CSVs refer to).  Families:
//   a4w4   : A e2m1 [M,K/2] row-major,  B e2m1 preshuffled (or row-major)
//   a8w4   : A e4m3 [M,K] (row-major or preshuffled), B e2m1 preshuffled
//   a16w16 : A bf16 [M,K], B bf16 [N,K] (row-major or preshuffled)
// Each family has tile instances (LDS double-buffered, 4 waves) and skinny
// instances (HBM streaming for small M, optional split-K over blocks).

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "gemm_registry.h"
#include "out_quant.h"

namespace aiter_amd {

std::string& last_error() {
    thread_local std::string msg;
    return msg;
}

int device_cu_count(int dev) {
    static std::mutex mu;
    static std::map<int, int> cache;
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    hipDeviceProp_t prop;
    AA_HIP(hipGetDeviceProperties(&prop, dev));
    cache[dev] = prop.multiProcessorCount;
    return prop.multiProcessorCount;
}

namespace {



std::vector<Instance>& registry() {
    static std::vector<Instance> reg;
    static std::once_flag once;
    std::call_once(once, [] {
        RegBuilder b{reg};
        b.part_mx();
        b.part_bf16<false>();
        b.part_bf16<true>();
        b.part_persist_split();
        b.part_rest();
        b.part_direct();
        b.part_late();
    });
    return reg;
}

const Instance* find_by_name(const std::string& nm) {
    for (auto& in : registry())
        if (in.name == nm) return &in;
    return nullptr;
}

const Instance* find_by_id(int id) {
    auto& r = registry();
    return (id >= 0 && id < (int)r.size()) ? &r[id] : nullptr;
}

bool variant_ok(const Instance& in, Family f, const Variant& v) {
    return in.fam == f && in.var.a_pre == v.a_pre && in.var.b_pre == v.b_pre && in.var.out_f32 == v.out_f32;
}

// Split-K factor for a skinny launch: split only when the 16-column blocks
// cannot cover the CUs, keeping >= 32 k-steps (8 per wave) per split.
int skinny_splits(int n_blocks, int k_steps, int cus) {
    int s = 1;
    while (n_blocks * s < cus && k_steps / (s * 2) >= 32) s *= 2;
    return s;
}

// Split-K factor for a split tile launch: enough splits for about one
// workgroup per CU, keeping >= 8 stages per split.
int tile_splits(int tiles, int stages, int cus) {
    int s = 1;
    while (tiles * s * 2 <= cus && stages / (s * 2) >= 8) s *= 2;
    return s;
}

// Heuristic choice among tile instances (reference heuristic idea:
// csrc/py_itfs_cu/asm_gemm_a4w4.cu:81-152 — fewest rounds of tiles over the
// CUs, then higher tile compute/memory ratio).
const Instance* heuristic(Family f, const Variant& v, int M, int N, int K, int cus, int* splits) {
    *splits = 1;
    const int ksteps = K / (f == kA16W16 ? 32 : 128);
    if (M <= 32) {
        const int mf = M <= 16 ? 1 : 2;
        const int nblk = (N + 15) / 16;
        const int s = skinny_splits(nblk, ksteps, cus);
        // 32-column workgroups when M > 8 and they still cover ~3/4 of the
        // CUs: each A fragment then serves two B blocks (A's L2 traffic per
        // B byte halves); measured 4.3 -> 4.0 us at M=16 and 5.4 -> 4.4 us at
        // M=32 for N=7168, K=2048, and no gain at M=1
        auto pick = [&](int bn, bool split) {
            const Instance* got = nullptr;
            for (auto& in : registry())
                if (in.skinny && variant_ok(in, f, v) && in.bm == 16 * mf && in.bn == bn && in.split == split &&
                    (!got || in.rank > got->rank))
                    got = &in;
            return got;
        };
        if (M > 8 && s == 1 && (N + 31) / 32 * 4 >= cus * 3)
            if (const Instance* in = pick(32, false)) return in;
        if (const Instance* in = pick(16, s > 1)) {
            *splits = s;
            return in;
        }
    }
    // time ~ rounds of tiles x per-tile time, and a tile's time per K step
    // grows like BM + BN (operand bytes) while its work grows like BM * BN:
    // minimise rounds * (BM + BN); on ties the larger tile
    const Instance* best = nullptr;
    long best_cost = 1L << 40;
    long best_tiles = 0;
    for (auto& in : registry()) {
        if (in.skinny || in.persistent || in.split || !variant_ok(in, f, v)) continue;   // tuned tables only
        const long tiles = (long)((M + in.bm - 1) / in.bm) * ((N + in.bn - 1) / in.bn);
        const long rounds = (tiles + cus - 1) / cus;
        const long cost = rounds * (in.bm + in.bn);
        if (cost < best_cost || (cost == best_cost && tiles < best_tiles)) {
            best = &in;
            best_cost = cost;
            best_tiles = tiles;
        }
    }
    // a grid that leaves most CUs idle splits K when the tile has a split form
    const int nst = K / (f == kA16W16 ? 64 : 256);
    if (best && best_tiles * 2 <= cus && nst >= 16) {
        for (auto& in : registry())
            if (!in.skinny && in.split && !in.persistent && in.bm == best->bm && in.bn == best->bn &&
                variant_ok(in, f, v)) {
                *splits = 0;   // the launcher picks the split count
                return &in;
            }
    }
    return best;
}

// The block tile a kernel of the reference is built for, read from its name.
struct RefTile {
    int tm = 0, tn = 0;
    bool split = false;
};

// Parses "<a>x<b>[x<c>...]" starting at s[i]; returns the number of fields.
int parse_dims(const std::string& s, size_t i, int* out, int max_fields) {
    int n = 0;
    while (n < max_fields && i < s.size() && isdigit((unsigned char)s[i])) {
        int v = 0;
        while (i < s.size() && isdigit((unsigned char)s[i])) v = v * 10 + (s[i++] - '0');
        out[n++] = v;
        if (i < s.size() && s[i] == 'x') ++i;
        else break;
    }
    return n;
}

// Reference kernel names carry their tile:
//  * ASM manifests (hsa/gfx950/f4gemm/f4gemm_bf16_per1x32Fp4.csv,
//    hsa/gfx950/bf16gemm/*.csv): mangled "_ZN5aiter<len><stem>_<tM>x<tN>[_tags]E",
//    split-K kernels tagged "splitk";
//  * CK A4W4 instances (csrc/ck_gemm_a4w4_blockscale/gemm_a4w4_blockscale_common.py:27-58):
//    "a4w4_blockscale_<block>x<tM>x<tN>x<tK>_...".
bool parse_reference_tile(const std::string& nm, RefTile* t) {
    static const std::string ck = "a4w4_blockscale_";
    if (nm.compare(0, ck.size(), ck) == 0) {
        int d[4];
        if (parse_dims(nm, ck.size(), d, 4) != 4 || d[1] <= 0 || d[2] <= 0) return false;
        t->tm = d[1];
        t->tn = d[2];
        t->split = false;
        return true;
    }
    if (nm.compare(0, 3, "_ZN") != 0 || nm.back() != 'E') return false;
    // the first "_<digits>x<digits>" field after the namespace prefix
    for (size_t i = nm.find('_', 3); i != std::string::npos && i + 1 < nm.size(); i = nm.find('_', i + 1)) {
        int d[2];
        if (parse_dims(nm, i + 1, d, 2) == 2 && d[0] > 0 && d[1] > 0) {
            t->tm = d[0];
            t->tn = d[1];
            t->split = nm.find("splitk") != std::string::npos;
            return true;
        }
    }
    return false;
}

// opus a16w16 kernel ids (csrc/opus_gemm/opus_gemm_common.py:238-513): the
// tile of each kid.  Offsets: +1000 no-OOB mirror, +2000/+3000/+4000 cache
// policy variants of kids 4-9, +5000 the >4 GiB-safe form; 4-9 mfma tiles,
// 200-223 flatmm split-K tiles, 300-315 persistent tiles, 1400-1404 mono
// tiles.  Returns false for ids outside the gfx950 table.
bool decode_opus_kid(int kid, RefTile* t) {
    if (kid < 0 || kid >= 10000) return false;   // >= 10000: the gfx942 table
    int k = kid >= 5000 ? kid - 5000 : kid;
    static const int mono[5][2] = {{192, 256}, {128, 256}, {192, 128}, {128, 128}, {64, 128}};
    if (k >= 1400 && k <= 1404) {
        t->tm = mono[k - 1400][0];
        t->tn = mono[k - 1400][1];
        t->split = false;
        return true;
    }
    if (k >= 2000) {
        if (k % 1000 < 4 || k % 1000 > 9) return false;
        k %= 1000;   // cache-policy variants (and their no-OOB mirrors) of kids 4-9
    } else if (k >= 1000) {
        k -= 1000;
    }
    static const int mfma[6][2] = {{128, 256}, {256, 128}, {128, 128}, {256, 128}, {128, 256}, {256, 256}};
    static const int flat[24][2] = {{64, 64},  {32, 32}, {32, 32}, {32, 64}, {32, 128}, {64, 32},
                                    {64, 32},  {128, 32}, {64, 64}, {256, 32}, {32, 256}, {32, 96},
                                    {32, 96},  {32, 96}, {64, 96}, {64, 96}, {64, 96},  {96, 32},
                                    {96, 32},  {96, 32}, {96, 64}, {96, 64}, {96, 64},  {96, 96}};
    static const int pers[4][2] = {{256, 256}, {128, 256}, {256, 128}, {128, 128}};
    if (k >= 4 && k <= 9) {
        t->tm = mfma[k - 4][0];
        t->tn = mfma[k - 4][1];
        t->split = false;
    } else if (k >= 200 && k <= 223) {
        t->tm = flat[k - 200][0];
        t->tn = flat[k - 200][1];
        t->split = true;
    } else if (k >= 300 && k <= 315) {
        t->tm = pers[(k - 300) % 4][0];
        t->tn = pers[(k - 300) % 4][1];
        t->split = false;
    } else {
        return false;
    }
    return true;
}

// This library's instance for a reference tile: the one-tile kernel of the
// same block shape (its split-K form for a split-K reference kernel) when
// there is one and M is beyond the skinny range; otherwise nullptr, and the
// caller takes its own heuristic choice for the shape (the reference's
// tiles were tuned for the reference's kernels; a tile this library lacks is
// not approximated by a neighbour).
const Instance* reference_tile_instance(const RefTile& t, Family f, const Variant& v, int64_t M) {
    if (M <= 32) return nullptr;
    for (int pass = 0; pass < 2; ++pass) {
        const bool want_split = pass == 0 ? t.split : false;
        if (pass == 1 && !t.split) break;
        for (auto& in : registry())
            if (!in.skinny && !in.persistent && in.split == want_split && in.bm == t.tm && in.bn == t.tn &&
                variant_ok(in, f, v))
                return &in;
    }
    return nullptr;
}

// A kernel name: this library's instance of that name (even when it does
// not fit the call: the caller reports that), or for a reference kernel name
// the instance reference_tile_instance picks (nullptr: the heuristic).
// *known is false when the name is neither.
const Instance* resolve_name(const std::string& nm, Family f, const Variant& v, int64_t M, bool* known) {
    *known = true;
    if (const Instance* in = find_by_name(nm)) return in;
    RefTile t;
    if (!parse_reference_tile(nm, &t)) {
        *known = false;
        return nullptr;
    }
    return reference_tile_instance(t, f, v, M);
}

__global__ __launch_bounds__(256) void fill_byte_kernel(uint8_t* p, int64_t n, int v) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16;
    const int w = v * 0x01010101;
    if (i + 16 <= n) *reinterpret_cast<i32x4_t*>(p + i) = i32x4_t{w, w, w, w};
    else
        for (int64_t j = i; j < n; ++j) p[j] = (uint8_t)v;
}

// ---- per-(device, stream) f32 workspace for split-K ----------------------
struct WsKey {
    int dev;
    hipStream_t st;
    // 0: split-K partials, 1: low-precision-output f32 tile, 2: unit scales,
    // 3 / 4: x / w scales of a fused call shuffled, 5: tile counters (kCounterSlot)
    int slot;
    bool operator<(const WsKey& o) const {
        return dev != o.dev ? dev < o.dev : (st != o.st ? st < o.st : slot < o.slot);
    }
};
constexpr int kCounterSlot = 5;
struct WsVal {
    float* ptr = nullptr;
    size_t bytes = 0;
};

std::mutex& workspace_mutex() {
    static std::mutex mu;
    return mu;
}
std::map<WsKey, WsVal>& workspace_map() {
    static std::map<WsKey, WsVal> ws;
    return ws;
}

float* workspace(int dev, hipStream_t st, size_t bytes, int slot = 0) {
    std::lock_guard<std::mutex> lk(workspace_mutex());
    auto& ws = workspace_map();
    WsVal& w = ws[{dev, st, slot}];
    if (w.bytes < bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        AA_HIP(hipStreamIsCapturing(st, &cs));
        AA_CHECK(cs == hipStreamCaptureStatusNone, "library workspace slot ", slot,
                 " must be sized before graph capture (split-K: gemm_workspace_reserve; low-precision outputs: "
                 "one eager call of the same shape)");
        if (w.ptr) {
            AA_HIP(hipStreamSynchronize(st));
            AA_HIP(hipFree(w.ptr));
        }
        AA_HIP(hipMalloc(&w.ptr, bytes));
        w.bytes = bytes;
        // counters start at zero; their users set them back to zero (never
        // during graph capture: allocation is refused there)
        if (slot == kCounterSlot) AA_HIP(hipMemsetAsync(w.ptr, 0, bytes, st));
    }
    return w.ptr;
}

struct GemmCall {
    Family fam;
    Variant var;
    const aiter_tensor_t *A, *B, *As, *Bs, *out, *bias;
    float alpha, beta;
    const char* kernel_name;
    int kernel_id;    // < 0: use name / heuristic
    int log2_split;   // < 0: heuristic
    // > 0: this many K splits (a literal KBatch, overrides log2_split)
    int split_count = 0;
    // batch > 1: one launch with gridDim.z = batch; A, B, out describe batch 0
    // and the strides (bytes; bias in elements) step to the next batch
    int batch = 1;
    int64_t bs_a = 0, bs_b = 0, bs_d = 0, bs_bias = 0;
    // packed e2m1 output through the 256x256 persistent kernel's epilogue:
    // `out` then describes [M, N] elements (row stride in elements) at the
    // packed bytes, with a bf16 dtype tag; only mxfp4_gemm_asm sets it
    bool out_fp4 = false;
    // an opus kernel id of the reference, decoded to its tile (tm > 0)
    RefTile ref_tile;
    // caller-free scratch (gemm_a4w4_asm_noalloc): used instead of the
    // library workspace for split-K partials; nothing is allocated
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // output operation fused into the epilogue (fused_gemm_afp4wfp4_*); the
    // persistent kernels do not carry it, their one-tile twins do
    EpiOp epi{};
    // plan only: a non-split skinny call stores its prepared parameters
    // here instead of launching (the caller launches them in a combined grid)
    GemmParams* capture = nullptr;
};

// split-K partial buffer of a call: the call's scratch when it brings one
// (never grown: too small is an error), else the (device, stream) workspace
float* split_buffer(const GemmCall& c, int dev, hipStream_t st, size_t need) {
    if (c.scratch) {
        AA_CHECK(need <= c.scratch_bytes, "split-K partials need ", need, " bytes, more than the ", c.scratch_bytes,
                 "-byte scratch of the no-allocation entry point");
        return static_cast<float*>(c.scratch);
    }
    return workspace(dev, st, need);
}

// rows [m0, m0 + rows) of a tensor viewed as 2-D (row-major rows of its
// last dimension), as a 2-D descriptor
aiter_tensor_t row_slice(const aiter_tensor_t* t, int64_t m0, int64_t rows, const char* what) {
    const int64_t ld = row_stride_2d(t, what);
    aiter_tensor_t v = *t;
    v.ptr = static_cast<uint8_t*>(t->ptr) + m0 * ld * (int64_t)dtype_size(t->dtype);
    v.ndim = 2;
    v.shape[0] = rows;
    v.shape[1] = cols_2d(t);
    v.strides[0] = ld;
    v.strides[1] = 1;
    v.numel = (size_t)(rows * cols_2d(t));
    return v;
}

void run_gemm(const GemmCall& c, hipStream_t stream);

// The kernels address A, out and the scales through 32-bit byte offsets: a
// call whose output or A reaches 2 GiB runs as row chunks of a multiple of
// 256 rows (shuffled scales keep whole 32-row groups contiguous, so a chunk's
// A scales start m0 * K/32 bytes in).  Returns false when no chunking is needed.
bool run_gemm_chunked(const GemmCall& c, hipStream_t stream) {
    const int64_t M = rows_2d(c.A);
    const int64_t orow = row_stride_2d(c.out, "out") * (int64_t)dtype_size(c.out->dtype);
    const int64_t arow = row_stride_2d(c.A, "A") * (int64_t)dtype_size(c.A->dtype);
    const int64_t lim = (int64_t)1 << 31;
    if (M <= 256 || (M * orow < lim && M * arow < lim)) return false;
    AA_CHECK(c.batch == 1 && !c.capture && !c.out_fp4 && !c.epi.kind,
             "a GEMM with 2 GiB or more of output or A runs in row chunks: no batch, fused epilogue or fp4 output");
    const int64_t chunk = std::min((lim - 1) / orow, (lim - 1) / arow) / 256 * 256;
    AA_CHECK(chunk >= 256, "rows of out or A too long for 32-bit offsets");
    const int64_t kb = c.fam == kA16W16 ? 0 : (c.fam == kA4W4 ? cols_2d(c.A) * 2 : cols_2d(c.A)) / 32;
    for (int64_t m0 = 0; m0 < M; m0 += chunk) {
        const int64_t rows = std::min(chunk, M - m0);
        aiter_tensor_t a = row_slice(c.A, m0, rows, "A"), o = row_slice(c.out, m0, rows, "out"), as{}, bias{};
        GemmCall cc = c;
        cc.A = &a;
        cc.out = &o;
        if (c.As) {
            as = *c.As;
            as.ptr = static_cast<uint8_t*>(c.As->ptr) + m0 * kb;
            as.ndim = 1;
            as.shape[0] = (int64_t)c.As->numel - m0 * kb;
            as.strides[0] = 1;
            as.numel = (size_t)as.shape[0];
            cc.As = &as;
        }
        if (c.bias && rows_2d(c.bias) > 1) {
            bias = row_slice(c.bias, m0, rows, "bias");
            cc.bias = &bias;
        }
        run_gemm(cc, stream);
    }
    return true;
}

void run_gemm(const GemmCall& c, hipStream_t stream) {
    check_tensor(c.A, "A", 2);
    check_tensor(c.B, "B", 2);
    check_tensor(c.out, "out", 2);
    if (run_gemm_chunked(c, stream)) return;
    const bool scaled = c.fam != kA16W16;
    const int64_t M = rows_2d(c.A), N = rows_2d(c.B);
    int64_t K;
    if (c.fam == kA4W4) {
        AA_CHECK(is_byte_type(c.A->dtype) && is_byte_type(c.B->dtype), "A and B must be fp4x2/u8");
        K = cols_2d(c.A) * 2;
        AA_CHECK(cols_2d(c.B) * 2 == K, "B K dim ", cols_2d(c.B) * 2, " != A K dim ", K);
    } else if (c.fam == kA8W4) {
        AA_CHECK(is_byte_type(c.A->dtype) && is_byte_type(c.B->dtype), "A must be fp8, B fp4x2");
        K = cols_2d(c.A);
        AA_CHECK(cols_2d(c.B) * 2 == K, "B K dim ", cols_2d(c.B) * 2, " != A K dim ", K);
    } else {
        AA_CHECK(c.A->dtype == AITER_DTYPE_bf16 && c.B->dtype == AITER_DTYPE_bf16,
                 "A and B must be bf16 (got ", dtype_name(c.A->dtype), ", ", dtype_name(c.B->dtype), ")");
        K = cols_2d(c.A);
        AA_CHECK(cols_2d(c.B) == K, "B K dim ", cols_2d(c.B), " != A K dim ", K);
    }
    AA_CHECK(c.var.out_f32 ? c.out->dtype == AITER_DTYPE_fp32 : c.out->dtype == AITER_DTYPE_bf16,
             "unsupported output dtype ", dtype_name(c.out->dtype));
    AA_CHECK(cols_2d(c.out) == N, "out has ", cols_2d(c.out), " columns, expected N = ", N);
    AA_CHECK(rows_2d(c.out) >= M, "out has ", rows_2d(c.out), " rows, expected >= M = ", M);
    const int kgran = scaled ? 256 : 64;
    AA_CHECK(K % kgran == 0, "K = ", K, " must be a multiple of ", kgran);
    AA_CHECK(N % 16 == 0, "N = ", N, " must be a multiple of 16");
    if (M == 0 || N == 0) return;
    AA_CHECK(M < (1LL << 31) && N < (1LL << 31), "M/N too large");

    const int64_t elem = (c.fam == kA16W16) ? 2 : 1;
    // the MX kernels address A, B and the scales through 32-bit buffer offsets
    if (scaled)
        AA_CHECK(M * row_stride_2d(c.A, "A") < (1LL << 31) && N * row_stride_2d(c.B, "B") < (1LL << 31),
                 "A and B must each be smaller than 2 GiB");
    GemmParams p{};
    p.A = static_cast<const uint8_t*>(c.A->ptr);
    p.B = static_cast<const uint8_t*>(c.B->ptr);
    p.lda = row_stride_2d(c.A, "A") * elem;
    p.ldb = row_stride_2d(c.B, "B") * elem;
    if (c.var.a_pre) AA_CHECK(M % 16 == 0 && p.lda == cols_2d(c.A) * elem, "preshuffled A needs M%16==0 and contiguity");
    if (c.var.b_pre) AA_CHECK(p.ldb == cols_2d(c.B) * elem, "preshuffled B must be contiguous");
    AA_CHECK(p.lda % 16 == 0 && p.ldb % 16 == 0 && ((uintptr_t)p.A & 15) == 0 && ((uintptr_t)p.B & 15) == 0,
             "A/B rows must be 16-byte aligned");
    p.D = c.out->ptr;
    p.ldd = row_stride_2d(c.out, "out");
    AA_CHECK((p.ldd * (c.var.out_f32 ? 4 : 2)) % 16 == 0 && ((uintptr_t)p.D & 15) == 0,
             "out rows must be 16-byte aligned");
    AA_CHECK(M * p.ldd * (c.var.out_f32 ? 4 : 2) < (1LL << 31), "out must be smaller than 2 GiB");
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.alpha = c.alpha;
    p.beta = c.beta;
    p.epi = c.epi;
    if (c.bias) {
        check_tensor(c.bias, "bias");
        AA_CHECK(c.bias->dtype == AITER_DTYPE_fp32, "bias must be f32");
        AA_CHECK(cols_2d(c.bias) == N, "bias last dim must be N");
        const int64_t br = rows_2d(c.bias);
        AA_CHECK(br == 1 || br >= M, "bias must be [N], [1,N] or [M,N]");
        p.bias = static_cast<const float*>(c.bias->ptr);
        p.ld_bias = br == 1 ? 0 : row_stride_2d(c.bias, "bias");
        AA_CHECK(p.ld_bias % 4 == 0 && ((uintptr_t)p.bias & 15) == 0, "bias rows must be 16-byte aligned");
    }
    if (scaled) {
        check_tensor(c.As, "A_scale", 1);
        check_tensor(c.Bs, "B_scale", 1);
        const int64_t kb = K / 32;  // multiple of 8 since K % 256 == 0
        p.As = static_cast<const uint8_t*>(c.As->ptr);
        p.Bs = static_cast<const uint8_t*>(c.Bs->ptr);
        p.sa_stride = c.As->ndim >= 2 ? row_stride_2d(c.As, "A_scale") : kb;
        p.sb_stride = c.Bs->ndim >= 2 ? row_stride_2d(c.Bs, "B_scale") : kb;
        AA_CHECK(p.sa_stride == kb && p.sb_stride == kb,
                 "shuffled scales must be contiguous with pad8(K/32) = ", kb, " bytes per row");
        const int64_t arows = (int64_t)c.As->numel / kb, brows = (int64_t)c.Bs->numel / kb;
        AA_CHECK(arows >= (M + 31) / 32 * 32, "A_scale has ", arows, " rows, need >= pad32(M) = ", (M + 31) / 32 * 32);
        AA_CHECK(brows >= (N + 31) / 32 * 32, "B_scale has ", brows, " rows, need >= pad32(N) = ", (N + 31) / 32 * 32);
        p.sa_groups = (int)(arows / 32);
        p.sb_groups = (int)(brows / 32);
    }

    int dev = c.A->device_id;
    if (dev < 0) AA_HIP(hipGetDevice(&dev));
    const int cus = device_cu_count(dev);

    const Instance* inst = nullptr;
    p.bs_a = c.bs_a;
    p.bs_b = c.bs_b;
    p.bs_d = c.bs_d;
    p.bs_bias = c.bs_bias;
    AA_CHECK(c.batch >= 1 && c.batch < 65536, "batch must be in [1, 65535]");
    const bool batched = c.batch > 1;   // one-pass, one-tile-per-workgroup kernels only
    int splits = 1;
    if (c.kernel_id >= 0) {
        inst = find_by_id(c.kernel_id);
        AA_CHECK(inst && variant_ok(*inst, c.fam, c.var), "kernel id ", c.kernel_id, " does not fit this GEMM");
    } else if (c.kernel_name && c.kernel_name[0]) {
        bool known = false;
        inst = resolve_name(c.kernel_name, c.fam, c.var, M, &known);
        AA_CHECK(known, "unknown kernel name '", c.kernel_name, "'");
        if (inst) AA_CHECK(variant_ok(*inst, c.fam, c.var), "kernel '", c.kernel_name, "' does not fit this GEMM");
    } else if (c.ref_tile.tm > 0) {
        inst = reference_tile_instance(c.ref_tile, c.fam, c.var, M);
    }
    const int ksteps = (int)(K / (scaled ? 128 : 32));
    if (!inst) {
        inst = heuristic(c.fam, c.var, (int)M, (int)N, (int)K, cus, &splits);
        AA_CHECK(inst, "no kernel instance for this GEMM");
    } else if (inst->skinny && inst->split) {
        splits = skinny_splits((int)((N + 15) / 16), ksteps, cus);
    }
    // requested split count (0: the launcher chooses)
    const int req_splits = c.split_count > 0 ? c.split_count : (c.log2_split >= 0 ? 1 << std::min(c.log2_split, 16) : 0);
    if (inst->skinny && inst->split && req_splits > 0) splits = req_splits;
    if (inst->skinny) AA_CHECK(M <= inst->bm, "skinny kernel ", inst->name, " covers M <= ", inst->bm);
    AA_CHECK(!c.capture || (inst->skinny && !inst->split && !inst->stream_k && !batched),
             "planned calls take non-split skinny kernels");

    if (!inst->skinny) {
        p.tiles_m = (int)((M + inst->bm - 1) / inst->bm);
        p.tiles_n = (int)((N + inst->bn - 1) / inst->bn);
        AA_CHECK(M >= 16 || !c.var.a_pre, "preshuffled A needs M >= 16");
        const int tiles = p.tiles_m * p.tiles_n;
        if (inst->split) {
            // split-K tile: stages of K over gridDim.y, f32 slices, then a sum
            const int nst = (int)(K / (scaled ? 256 : 64));
            int sp = req_splits > 0 ? req_splits : tile_splits(tiles, nst, cus);
            if (batched) sp = 1;
            sp = std::max(1, std::min(sp, nst));
            p.k_steps_per_split = (nst + sp - 1) / sp;
            sp = (nst + p.k_steps_per_split - 1) / p.k_steps_per_split;
            if (sp > 1) {
                const size_t need = (size_t)sp * M * N * sizeof(float);
                p.ws = split_buffer(c, dev, stream, need);
                inst->fn(p, dim3(tiles, sp), stream);
                const unsigned blocks = (unsigned)(((int64_t)M * N / 4 + 255) / 256);
                if (c.var.out_f32)
                    splitk_reduce_kernel<true><<<dim3(blocks), 256, 0, stream>>>(p, sp);
                else
                    splitk_reduce_kernel<false><<<dim3(blocks), 256, 0, stream>>>(p, sp);
                AA_HIP(hipGetLastError());
                return;
            }
            // one split: the same tile without the split
            const Instance* twin = nullptr;
            for (auto& in : registry())
                if (!in.skinny && !in.split && !in.persistent && in.bm == inst->bm && in.bn == inst->bn &&
                    variant_ok(in, c.fam, c.var))
                    twin = &in;
            AA_CHECK(twin, "no non-split twin of ", inst->name);
            inst = twin;
        }
        // the persistent kernels address A and B through whole-tensor 32-bit
        // buffer offsets
        const bool big = M * p.lda >= (1LL << 31) || N * p.ldb >= (1LL << 31);
        if (inst->persistent && (p.bias || batched || big || c.epi.kind)) {
            // the persistent epilogue has no bias term: its one-tile-per-workgroup twin
            const Instance* twin = nullptr;
            for (auto& in : registry())
                if (!in.skinny && !in.persistent && in.fam == inst->fam && in.bm == inst->bm && in.bn == inst->bn &&
                    variant_ok(in, c.fam, c.var))
                    twin = &in;
            AA_CHECK(twin, "no non-persistent twin of ", inst->name);
            inst = twin;
        }
        if (c.out_fp4) {
            AA_CHECK(inst->persistent && inst->fam == kA4W4 && inst->bm == 256 && inst->bn == 256 && c.var.b_pre &&
                         !c.var.out_f32 && !p.bias && !batched,
                     "packed-fp4 epilogue: only the 256x256 persistent A4W4 tile, no bias or batch");
            gemm_flat_persist_kernel<kFp4, 256, false, true, true, false>
                <<<dim3(std::min(tiles, cus), 1, 1), 256, 0, stream>>>(p);
            AA_HIP(hipGetLastError());
            return;
        }
        inst->fn(p, dim3(inst->persistent ? std::min(tiles, cus) : tiles, 1, c.batch), stream);
    } else {
        // the skinny kernels split K in k-pairs (one scale dword each)
        const int kpairs = ksteps / 2;
        if (inst->stream_k) {
            // up to one workgroup per CU over the (column block, k-pair)
            // units, and about 8 ranges per block at most (the range that sums
            // a block loads the others' partials 8 at a time); two partial
            // slots per workgroup, one arrival counter per block
            AA_CHECK(!batched && !c.scratch, "stream-K skinny kernel ", inst->name, ": no batch, no caller scratch");
            const int64_t nblk = (N + inst->bn - 1) / inst->bn;
            const int grid = (int)std::min<int64_t>(std::min<int64_t>(cus, nblk * 8), nblk * kpairs);
            p.k_steps_per_split = kpairs;
            p.ws = split_buffer(c, dev, stream, (size_t)2 * grid * inst->bm * inst->bn * sizeof(float));
            p.cnt = lib_counters(dev, stream, (size_t)nblk);
            inst->fn(p, dim3((unsigned)grid), stream);
            AA_HIP(hipGetLastError());
            return;
        }
        splits = batched ? 1 : std::max(1, std::min(splits, kpairs));
        p.k_steps_per_split = (kpairs + splits - 1) / splits;
        splits = (kpairs + p.k_steps_per_split - 1) / p.k_steps_per_split;
        const dim3 grid((unsigned)((N + inst->bn - 1) / inst->bn), (unsigned)splits);
        if (inst->split && splits > 1) {
            const int64_t n4 = (int64_t)M * N;
            // f32 output with nothing to apply after the sum (no bias, alpha
            // 1, no fused operation) and rows of exactly N: the partials add
            // straight into the zeroed output, no workspace and no finish launch
            const bool direct = c.var.out_f32 && p.ldd == N && !p.bias && p.alpha == 1.0f && !c.epi.kind;
            p.ws = direct ? static_cast<float*>(p.D) : split_buffer(c, dev, stream, (size_t)n4 * sizeof(float));
            fill_zero_kernel<><<<dim3((unsigned)((n4 / 4 + 255) / 256 + 1)), 256, 0, stream>>>(p.ws, n4);
            inst->fn(p, grid, stream);
            if (direct) {
                // summed in place
            } else if (c.var.out_f32) {
                splitk_finish_kernel<true><<<dim3((unsigned)((n4 / 4 + 255) / 256)), 256, 0, stream>>>(p);
            } else {
                splitk_finish_kernel<false><<<dim3((unsigned)((n4 / 4 + 255) / 256)), 256, 0, stream>>>(p);
            }
        } else if (inst->split) {
            // a split instance asked for one split runs its non-split twin
            // (the highest-ranked one, first registered among equals)
            const Instance* twin = nullptr;
            for (auto& in : registry())
                if (in.skinny && !in.split && variant_ok(in, c.fam, c.var) && in.bm == inst->bm &&
                    in.bn == inst->bn && (!twin || in.rank > twin->rank))
                    twin = &in;
            AA_CHECK(twin, "no non-split twin for ", inst->name);
            p.k_steps_per_split = kpairs;
            twin->fn(p, dim3(grid.x, 1, c.batch), stream);
        } else {
            p.k_steps_per_split = kpairs;
            if (c.capture) {
                *c.capture = p;
                return;
            }
            inst->fn(p, dim3(grid.x, 1, c.batch), stream);
        }
    }
    AA_HIP(hipGetLastError());
}

// ---- fixed scratch of the no-allocation entry point ----------------------
// One array per GPU, allocated with the code object when the library loads
// on that device; host code reaches it only through the device address
// hipGetSymbolAddress returns (the array's name is a host-side stand-in).
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// device address of `scratch` on `dev` (current device), looked up once
void* scratch_address(int dev) {
    static std::mutex mu;
    static std::map<int, void*> addr;
    std::lock_guard<std::mutex> lk(mu);
    auto it = addr.find(dev);
    if (it != addr.end()) return it->second;
    void* ptr = nullptr;
    AA_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    AA_CHECK(ptr, "no device address for the scratch array");
    addr[dev] = ptr;
    return ptr;
}

// ---- fused_gemm_afp4wfp4_* (aiter/ops/triton/gemm/fused/) ----

// plain e8m0 scales [rows, groups] (row stride in bytes) -> the shuffled
// layout of shuffle_scale (aiter/ops/shuffle.py:339-365), pad32(rows) rows,
// padding zero: output byte o of 32-row block i0 holds the scale of row
// i0*32 + 16*a + b, group 8*c + 4*d + e, o = i0*32*groups + 256c + 64e + 4b + 2d + a
__global__ __launch_bounds__(256) void plain_scale_shuffle_kernel(const uint8_t* src, int64_t src_stride, int rows,
                                                                  int groups, uint8_t* dst, int64_t total) {
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (o >= total) return;
    const int64_t blk = 32 * (int64_t)groups;
    const int i0 = (int)(o / blk);
    const int w0 = (int)(o - i0 * blk);
    const int c = w0 / 256, w = w0 % 256;
    const int e = w / 64, b = (w % 64) / 4, d = (w % 4) / 2, a = w % 2;
    const int r = i0 * 32 + a * 16 + b, g = c * 8 + d * 4 + e;
    dst[o] = r < rows ? src[(int64_t)r * src_stride + g] : 0;
}

// c1[m, d, S1 + j] = y[m, d, j] (bf16, y of any strides, c1 contiguous)
__global__ __launch_bounds__(256) void split_cat_copy_kernel(const uint16_t* y, int64_t ys0, int64_t ys1, int64_t ys2,
                                                             uint16_t* c1, int M, int D, int S1, int S3) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)M * D * S3) return;
    const int j = (int)(i % S3);
    const int64_t md = i / S3;
    const int d = (int)(md % D), m = (int)(md / D);
    c1[((int64_t)m * D + d) * (S1 + S3) + S1 + j] = y[m * ys0 + d * ys1 + j * ys2];
}

// contiguous [rows, cols] view of a tensor's bytes
aiter_tensor_t flat_view(const aiter_tensor_t* t, int64_t rows, int64_t cols, const char* what) {
    check_tensor(t, what);
    int64_t expect = 1;
    for (int d = t->ndim - 1; d >= 0; --d) {
        AA_CHECK(t->shape[d] == 1 || t->strides[d] == expect, what, " must be contiguous");
        expect *= t->shape[d];
    }
    AA_CHECK((int64_t)t->numel == rows * cols, what, " has ", t->numel, " elements, expected ", rows, " x ", cols);
    aiter_tensor_t v = *t;
    v.ndim = 2;
    v.shape[0] = rows;
    v.shape[1] = cols;
    v.strides[0] = cols;
    v.strides[1] = 1;
    return v;
}

// e8m0 scales of a fused call as the GEMM takes them: shuffled tensors (any
// shape over the shuffled bytes, e.g. the Triton [R/32, K] view) are viewed
// as [bytes / (K/32), K/32]; plain [R, K/32] tensors are shuffled into
// workspace slot `slot` first
aiter_tensor_t fused_scales(const aiter_tensor_t* sc, bool shuffled, int64_t R, int64_t K, int dev, hipStream_t st,
                            int slot, const char* what) {
    const int64_t kb = K / 32;
    check_tensor(sc, what);
    AA_CHECK(is_byte_type(sc->dtype), what, " must be e8m0 bytes");
    if (shuffled) {
        AA_CHECK((int64_t)sc->numel % kb == 0, what, " (shuffled) has ", sc->numel, " bytes, not a multiple of K/32");
        return flat_view(sc, (int64_t)sc->numel / kb, kb, what);
    }
    AA_CHECK(sc->ndim == 2 && rows_2d(sc) >= R && cols_2d(sc) == kb, what, " must be [", R, ", ", kb, "] (plain e8m0)");
    const int64_t stride = row_stride_2d(sc, what);
    const int64_t rows = (R + 31) / 32 * 32;
    uint8_t* dst = reinterpret_cast<uint8_t*>(workspace(dev, st, (size_t)(rows * kb), slot));
    const int64_t total = rows * kb;
    if (total > 0) {
        plain_scale_shuffle_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, st>>>(
            static_cast<const uint8_t*>(sc->ptr), stride, (int)R, (int)kb, dst, total);
        AA_HIP(hipGetLastError());
    }
    aiter_tensor_t v{};
    v.ptr = dst;
    v.numel = (size_t)total;
    v.ndim = 2;
    v.shape[0] = rows;
    v.shape[1] = kb;
    v.strides[0] = kb;
    v.strides[1] = 1;
    v.dtype = AITER_DTYPE_fp8_e8m0;
    v.device_id = sc->device_id;
    return v;
}

// A4W4 GEMM of a fused op: x [M, K/2], w [N, K/2] row-major or its
// shuffle_weight bytes (any shape, e.g. the Triton [N/16, K*8] view); with
// preshuffled w the w scales are shuffled and the x scales too when M >= 32
// (the Triton preshuffled ops' convention), otherwise both are plain
void fused_a4w4(const aiter_tensor_t* x, const aiter_tensor_t* w, const aiter_tensor_t* xs, const aiter_tensor_t* ws,
                bool preshuffled, const aiter_tensor_t* out, const aiter_tensor_t* bias, const EpiOp& epi,
                const char* kernel_name, hipStream_t st, GemmParams* capture = nullptr) {
    check_tensor(x, "x", 2);
    check_tensor(w, "w", 2);
    const int64_t M = rows_2d(x), K = cols_2d(x) * 2;
    AA_CHECK(K % 256 == 0, "K = ", K, " must be a multiple of 256");
    int64_t N;
    aiter_tensor_t wv;
    if (preshuffled) {
        AA_CHECK((int64_t)w->numel % (K / 2) == 0, "w (preshuffled) has ", w->numel, " bytes, not a multiple of K/2");
        N = (int64_t)w->numel / (K / 2);
        wv = flat_view(w, N, K / 2, "w");
    } else {
        N = rows_2d(w);
        AA_CHECK(cols_2d(w) * 2 == K, "w K dim ", cols_2d(w) * 2, " != x K dim ", K);
        wv = *w;
    }
    int dev = x->device_id;
    if (dev < 0) AA_HIP(hipGetDevice(&dev));
    const aiter_tensor_t xsv = fused_scales(xs, preshuffled && M >= 32, M, K, dev, st, 3, "x_scale");
    const aiter_tensor_t wsv = fused_scales(ws, preshuffled, N, K, dev, st, 4, "w_scale");
    GemmCall c{kA4W4, {false, preshuffled, false}, x, &wv, &xsv, &wsv, out, bias, 1.0f, 1.0f, kernel_name, -1, -1};
    c.epi = epi;
    c.capture = capture;
    run_gemm(c, st);
}

// one operand of mul_add: tensor broadcastable to [M, N] (f32 or bf16) or NULL
void mul_add_operand(const aiter_tensor_t* t, int64_t M, int64_t N, const void** ptr, int* bf16, int64_t* sm,
                     int64_t* sn, const char* what) {
    *ptr = nullptr;
    if (!t) return;
    check_tensor(t, what);
    AA_CHECK(t->dtype == AITER_DTYPE_fp32 || t->dtype == AITER_DTYPE_bf16, what, " must be f32 or bf16");
    *ptr = t->ptr;
    *bf16 = t->dtype == AITER_DTYPE_bf16;
    if (t->numel == 1) {
        *sm = *sn = 0;
        return;
    }
    AA_CHECK(t->ndim == 2, what, " must be a scalar or 2-D (broadcastable to [M, N])");
    AA_CHECK(t->shape[0] == M || t->shape[0] == 1, what, " has ", t->shape[0], " rows, expected ", M, " or 1");
    AA_CHECK(t->shape[1] == N || t->shape[1] == 1, what, " has ", t->shape[1], " columns, expected ", N, " or 1");
    *sm = t->shape[0] == 1 ? 0 : t->strides[0];
    *sn = t->shape[1] == 1 ? 0 : t->strides[1];
}

}  // namespace

void* lib_workspace(int dev, hipStream_t st, size_t bytes) { return workspace(dev, st, bytes); }
int* lib_counters(int dev, hipStream_t st, size_t count) {
    // at least 64K counters (256 KiB), so that gemm_workspace_reserve covers
    // the split-K calls of a later graph capture
    return reinterpret_cast<int*>(workspace(dev, st, std::max<size_t>(count, 65536) * sizeof(int), kCounterSlot));
}

}  // namespace aiter_amd

using namespace aiter_amd;

extern "C" {

int aiter_ctypes_abi_version(void) { return 2; }

const char* aiter_get_last_error(void) {
    return last_error().empty() ? nullptr : last_error().c_str();
}

void aiter_clear_last_error(void) { last_error().clear(); }

int getPaddedM(int M, int N, int K, int gl) {
    (void)K;
    int padded = M;
    if (gl == 0) {
        if (M <= 256) padded = (M + 15) / 16 * 16;
        else if (M <= 1024) padded = (M + 31) / 32 * 32;
        else if (M <= 4096) padded = (M + 63) / 64 * 64;
        else padded = (M + 127) / 128 * 128;
    } else if (gl == 1) {
        if (M > 8192 && N > 4096) {
            padded = 8192;
        } else {
            unsigned v = M <= 1 ? 1u : (unsigned)M;
            unsigned p2 = 1;
            while (p2 < v) p2 <<= 1;
            padded = (int)p2;
        }
    }
    return padded;
}

int gemm_a4w4_asm(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* A_scale,
                  aiter_tensor_t* B_scale, aiter_tensor_t* out, const char* kernelName,
                  aiter_tensor_t* bias, float alpha, float beta, int bpreshuffle, int log2_k_split,
                  aiter_stream_t stream) {
    return safe_call([&] {
        DeviceGuard g(A ? A->device_id : -1);
        GemmCall c{kA4W4, {false, bpreshuffle != 0, false}, A, B, A_scale, B_scale, out, bias,
                   alpha, beta, kernelName, -1, log2_k_split > 0 ? log2_k_split : -1};
        run_gemm(c, reinterpret_cast<hipStream_t>(stream));
    });
}

// gemm_a4w4_asm without any allocation: split-K partials go to the fixed
// per-GPU `scratch` array (kNoAllocScratchBytes), never to the library
// workspace; a call whose partials need more raises.  The array is shared by
// every call on the GPU and keeps the previous call's contents: the split
// kernels clear what they accumulate into with a fill kernel first, and
// calls that overlap on one GPU (two streams, two threads) race.
int gemm_a4w4_asm_noalloc(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* A_scale, aiter_tensor_t* B_scale,
                          aiter_tensor_t* out, const char* kernelName, aiter_tensor_t* bias, float alpha, float beta,
                          int bpreshuffle, int log2_k_split, aiter_stream_t stream) {
    return safe_call([&] {
        AA_CHECK(A, "A is NULL");
        DeviceGuard g(A->device_id);
        int dev = A->device_id;
        if (dev < 0) AA_HIP(hipGetDevice(&dev));
        GemmCall c{kA4W4, {false, bpreshuffle != 0, false}, A, B, A_scale, B_scale, out, bias,
                   alpha, beta, kernelName, -1, log2_k_split > 0 ? log2_k_split : -1};
        c.scratch = scratch_address(dev);
        c.scratch_bytes = kNoAllocScratchBytes;
        run_gemm(c, reinterpret_cast<hipStream_t>(stream));
    });
}

size_t gemm_a4w4_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

// gfx1250 f4gemm entry (aiter/ops/gemm_op_a4w4.py:290-304, dispatch :80-124):
// the output dtype picks the form: bf16 [M, N] (gemm_a4w4), fp4x2 [M, N/2]
// (e2m1 with conversion scale 1; the reference's packed-fp4 kernel ignores the
// input scales, op_tests/test_f4gemm.py:213-215, and so does this one: it runs
// with unit scales), or fp8 [M, N] + out_scale (MXFP8, per-128-column e8m0 in
// the packed layout).  e2m1 output on shapes whose 256x256 tiles fill the CUs
// (N % 32 == 0, no kernel named) is converted in the persistent kernel's
// epilogue; the other low-precision forms run the f32-output GEMM into a
// library-owned tile, then out_quant_kernel.
int mxfp4_gemm_asm(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* ScaleA, aiter_tensor_t* ScaleB,
                   aiter_tensor_t* out, aiter_tensor_t* out_scale, const char* kernelName, int a_preshuffle,
                   aiter_stream_t stream) {
    return safe_call([&] {
        check_tensor(A, "A", 2);
        check_tensor(B, "B", 2);
        check_tensor(out, "out", 2);
        DeviceGuard g(A->device_id);
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        AA_CHECK(!a_preshuffle, "mxfp4_gemm_asm: preshuffled A is a gfx1250 layout; pass a_preshuffle=0");
        const int odt = out->dtype;
        if (odt == AITER_DTYPE_bf16) {
            GemmCall c{kA4W4, {false, true, false}, A, B, ScaleA, ScaleB, out, nullptr, 1.0f, 0.0f, kernelName, -1, -1};
            run_gemm(c, st);
            return;
        }
        const bool fp8 = odt == AITER_DTYPE_fp8;
        AA_CHECK(fp8 || odt == AITER_DTYPE_fp4x2 || odt == AITER_DTYPE_u8,
                 "mxfp4_gemm_asm: out must be bf16, fp4x2 or fp8");
        const int64_t M = rows_2d(A), N = rows_2d(B), K = cols_2d(A) * 2;
        AA_CHECK(rows_2d(out) == M && cols_2d(out) == (fp8 ? N : N / 2) && out->strides[out->ndim - 1] == 1,
                 "mxfp4_gemm_asm: out must be [M, ", fp8 ? "N" : "N/2", "]");
        const int64_t out_stride = out->ndim >= 2 ? out->strides[out->ndim - 2] : cols_2d(out);
        AA_CHECK(N % 8 == 0 && out_stride % 4 == 0, "mxfp4_gemm_asm: N must be a multiple of 8");
        if (M == 0 || N == 0) return;
        if (fp8) {
            AA_CHECK(out_scale, "mxfp4_gemm_asm: MXFP8 output needs out_scale");
            AA_CHECK(N % 128 == 0 && M % 64 == 0, "mxfp4_gemm_asm: MXFP8 output needs N % 128 == 0 and M % 64 == 0");
            AA_CHECK(is_byte_type(out_scale->dtype) && (int64_t)out_scale->numel >= M * (N / 128),
                     "mxfp4_gemm_asm: out_scale must hold M * N / 128 e8m0 bytes");
        }
        aiter_tensor_t usa{}, usb{};
        const aiter_tensor_t *sa = ScaleA, *sb = ScaleB;
        if (!fp8) {
            // unit scales (byte 127): shuffled or not, every byte is 127
            const int64_t sn = (K / 32 + 7) / 8 * 8;
            const int64_t rows = (std::max(M, N) + 255) / 256 * 256;
            uint8_t* ones = reinterpret_cast<uint8_t*>(workspace(A->device_id, st, (size_t)(rows * sn), 2));
            fill_byte_kernel<<<(unsigned)((rows * sn / 16 + 255) / 256 + 1), 256, 0, st>>>(ones, rows * sn, 127);
            AA_HIP(hipGetLastError());
            for (aiter_tensor_t* u : {&usa, &usb}) {
                u->ptr = ones;
                u->ndim = 2;
                u->dtype = AITER_DTYPE_u8;
                u->device_id = A->device_id;
                u->strides[1] = 1;
                u->strides[0] = sn;
                u->shape[1] = sn;
            }
            usa.shape[0] = (M + 255) / 256 * 256;
            usb.shape[0] = (N + 255) / 256 * 256;
            usa.numel = usa.shape[0] * sn;
            usb.numel = usb.shape[0] * sn;
            sa = &usa;
            sb = &usb;
        }
        const bool fill = ((M + 255) / 256) * ((N + 255) / 256) >= device_cu_count(A->device_id);
        if (!fp8 && (!kernelName || !kernelName[0]) && fill && N % 32 == 0) {
            // e2m1 straight from the persistent 256x256 kernel's epilogue: no
            // f32 tile, no second pass
            aiter_tensor_t o{};
            o.ptr = out->ptr;
            o.ndim = 2;
            o.shape[0] = M;
            o.shape[1] = N;
            o.strides[0] = out_stride * 2;
            o.strides[1] = 1;
            o.numel = (size_t)(M * N);
            o.dtype = AITER_DTYPE_bf16;   // tag only: the fp4 epilogue writes packed bytes
            o.device_id = A->device_id;
            GemmCall c{kA4W4, {false, true, false}, A, B, sa, sb, &o, nullptr, 1.0f, 0.0f,
                       "a4w4_tile_256x256_persist", -1, -1};
            c.out_fp4 = true;
            run_gemm(c, st);
            return;
        }
        // f32 tile (library workspace), then the output quant
        float* tile = workspace(A->device_id, st, (size_t)M * N * sizeof(float), 1);
        aiter_tensor_t t{};
        t.ptr = tile;
        t.numel = (size_t)(M * N);
        t.ndim = 2;
        t.shape[0] = M;
        t.shape[1] = N;
        t.strides[0] = N;
        t.strides[1] = 1;
        t.dtype = AITER_DTYPE_fp32;
        t.device_id = A->device_id;
        // f32 tile: the persistent 256x256 kernel when its tiles fill the CUs
        // (8192^3: 297 vs 338 us through the heuristic's 128x256 tile), else
        // the heuristic
        const char* kn = kernelName;
        if ((!kn || !kn[0]) && fill)
            kn = "a4w4_tile_256x256_f32_persist";
        GemmCall c{kA4W4, {false, true, true}, A, B, sa, sb, &t, nullptr, 1.0f, 0.0f, kn, -1, -1};
        run_gemm(c, st);
        const int64_t n = M * (N / 8);
        const dim3 grid((unsigned)((n + 255) / 256));
        if (fp8)
            out_quant_kernel<true><<<grid, 256, 0, st>>>(tile, M, N, N, static_cast<uint8_t*>(out->ptr), out_stride,
                                                          static_cast<uint8_t*>(out_scale->ptr));
        else
            out_quant_kernel<false><<<grid, 256, 0, st>>>(tile, M, N, N, static_cast<uint8_t*>(out->ptr), out_stride,
                                                           nullptr);
        AA_HIP(hipGetLastError());
    });
}

int gemm_a4w4_blockscale(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* x_scale,
                         aiter_tensor_t* w_scale, aiter_tensor_t* Y, int splitK, int kernelId,
                         aiter_stream_t stream) {
    return safe_call([&] {
        DeviceGuard g(XQ ? XQ->device_id : -1);
        GemmCall c{kA4W4, {false, true, false}, XQ, WQ, x_scale, w_scale, Y, nullptr,
                   1.0f, 0.0f, nullptr, kernelId, splitK > 0 ? splitK : -1};
        run_gemm(c, reinterpret_cast<hipStream_t>(stream));
    });
}

int mxfp8_mxfp4_gemm_asm(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* ScaleA,
                         aiter_tensor_t* ScaleB, aiter_tensor_t* out, const char* kernelName,
                         int a_preshuffle, aiter_stream_t stream) {
    return safe_call([&] {
        DeviceGuard g(A ? A->device_id : -1);
        // the skinny path reads A row-major only
        GemmCall c{kA8W4, {a_preshuffle != 0, true, false}, A, B, ScaleA, ScaleB, out, nullptr,
                   1.0f, 0.0f, kernelName, -1, -1};
        if (a_preshuffle && rows_2d(A) <= 64) {
            // small-M heuristic is the skinny kernel, which needs row-major A
            AA_CHECK(!kernelName || !kernelName[0] || std::string(kernelName).find("tile") != std::string::npos,
                     "preshuffled A with M <= 64 supports tile kernels only");
            if (!kernelName || !kernelName[0]) c.kernel_name = "a8w4_tile_64x128_apre";
        }
        run_gemm(c, reinterpret_cast<hipStream_t>(stream));
    });
}

int gemm_a16w16_asm(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* out,
                    aiter_tensor_t* semaphore, aiter_tensor_t* bias, int splitK,
                    const char* kernelName, int bpreshuffle, aiter_stream_t stream) {
    (void)semaphore;
    return safe_call([&] {
        DeviceGuard g(A ? A->device_id : -1);
        // splitK is a literal split count, capped at 16
        // (csrc/py_itfs_cu/asm_gemm_a16w16.cu:111-114): 1 runs one pass; none
        // (<= 0) lets the launcher choose (the reference raises for 1 with a
        // split-K kernel; every split instance here has a one-pass twin)
        GemmCall c{kA16W16, {false, bpreshuffle != 0, out && out->dtype == AITER_DTYPE_fp32}, A, B,
                   nullptr, nullptr, out, bias, 1.0f, 1.0f, kernelName, -1, -1};
        if (splitK >= 1) c.split_count = std::min(splitK, 16);
        run_gemm(c, reinterpret_cast<hipStream_t>(stream));
    });
}

// [b, M, K] x [b, N, K] -> [b, M, N] (+ bias [N] or [b, N]) as one launch
// with gridDim.z = b: the 2-D descriptors of batch 0 plus batch strides (any
// strides with unit last-dimension stride, e.g. the reference test's [m, b, k]
// transposed layout)
// kernelId: with opus_kid an opus kernel id of the reference (decoded to its
// tile, decode_opus_kid), else an id of this library's table; < 0 heuristic.
static void opus_batched(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* Y, aiter_tensor_t* bias,
                         int kernelId, int splitK, hipStream_t st, bool opus_kid = false) {
    check_tensor(XQ, "XQ", 2);
    check_tensor(WQ, "WQ", 2);
    check_tensor(Y, "Y", 2);
    const int nd = XQ->ndim;
    const int64_t batch = nd == 3 ? XQ->shape[0] : 1;
    AA_CHECK(WQ->ndim == nd && Y->ndim == nd, "XQ, WQ, Y must have the same rank");
    AA_CHECK(nd == 2 || nd == 3, "opus a16w16 expects 2-D or 3-D tensors");
    if (nd == 3) AA_CHECK(WQ->shape[0] == batch && Y->shape[0] == batch, "batch mismatch");
    aiter_tensor_t a = *XQ, w = *WQ, y = *Y, bb{};
    auto slice0 = [&](aiter_tensor_t& t, const aiter_tensor_t* src) {
        if (nd == 3) {
            t.ndim = 2;
            t.shape[0] = src->shape[1];
            t.shape[1] = src->shape[2];
            t.strides[0] = src->strides[1];
            t.strides[1] = src->strides[2];
            t.numel = src->shape[1] * src->shape[2];
        }
    };
    slice0(a, XQ);
    slice0(w, WQ);
    slice0(y, Y);
    aiter_tensor_t* bptr = nullptr;
    int64_t bs_bias = 0;
    if (bias) {
        bb = *bias;
        if (bias->ndim == 2 && bias->shape[0] == batch && batch > 1) {
            bb.ndim = 1;
            bb.shape[0] = bias->shape[1];
            bb.strides[0] = bias->strides[1];
            bb.numel = bias->shape[1];
            bs_bias = bias->strides[0];
        }
        bptr = &bb;
    }
    GemmCall c{kA16W16, {false, false, Y->dtype == AITER_DTYPE_fp32}, &a, &w, nullptr, nullptr, &y, bptr,
               1.0f, 1.0f, nullptr, opus_kid ? -1 : kernelId, splitK > 0 ? splitK : -1};
    // the opus API passes a literal KBatch with its kernel id, <= 1 meaning
    // one pass (aiter/ops/opus/gemm_op_a16w16.py:488); the CK batched API
    // passes its log2
    if (opus_kid) {
        c.log2_split = -1;
        c.split_count = kernelId >= 0 ? std::max(splitK, 1) : 0;
    }
    if (opus_kid && kernelId >= 0)
        AA_CHECK(decode_opus_kid(kernelId, &c.ref_tile), "unknown opus kernel id ", kernelId,
                 " (not in the gfx950 opus table)");
    if (batch > 1) {
        c.batch = (int)batch;
        c.bs_a = XQ->strides[0] * 2;
        c.bs_b = WQ->strides[0] * 2;
        c.bs_d = Y->strides[0] * (int64_t)dtype_size(Y->dtype);
        c.bs_bias = bs_bias;
    }
    run_gemm(c, st);
}

int opus_gemm(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* Y, aiter_tensor_t* bias,
              aiter_stream_t stream) {
    return safe_call([&] {
        DeviceGuard g(XQ ? XQ->device_id : -1);
        opus_batched(XQ, WQ, Y, bias, -1, -1, reinterpret_cast<hipStream_t>(stream));
    });
}

int opus_gemm_a16w16_tune(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* Y,
                          aiter_tensor_t* bias, int kernelId, int splitK, aiter_stream_t stream) {
    return safe_call([&] {
        DeviceGuard g(XQ ? XQ->device_id : -1);
        opus_batched(XQ, WQ, Y, bias, kernelId, splitK, reinterpret_cast<hipStream_t>(stream), true);
    });
}

// CK batched bf16 API (aiter/ops/batched_gemm_op_bf16.py:28-36,127-134):
// XQ [B, M, K], WQ [B, N, K], Y [B, M, N] (bf16 or fp32), bias [N] or [B, N];
// one batched launch.  splitK is the log2 split request of the reference
// (ignored when the batch already fills the GPU: batched launches are one-pass).
int batched_gemm_bf16(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* Y, aiter_tensor_t* bias, int splitK,
                      aiter_stream_t stream) {
    return safe_call([&] {
        DeviceGuard g(XQ ? XQ->device_id : -1);
        AA_CHECK(XQ && XQ->ndim == 3, "batched_gemm_bf16: XQ must be [B, M, K]");
        opus_batched(XQ, WQ, Y, bias, -1, splitK, reinterpret_cast<hipStream_t>(stream));
    });
}

int batched_gemm_bf16_tune(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* Y, int kernelId, int splitK,
                           aiter_stream_t stream) {
    return safe_call([&] {
        DeviceGuard g(XQ ? XQ->device_id : -1);
        AA_CHECK(XQ && XQ->ndim == 3, "batched_gemm_bf16_tune: XQ must be [B, M, K]");
        opus_batched(XQ, WQ, Y, nullptr, kernelId, splitK, reinterpret_cast<hipStream_t>(stream));
    });
}

// ---- library-specific introspection (used by the Python tuner) ----------
int aiter_amd_num_kernels(void) { return (int)registry().size(); }

// Writes "id,name,family,skinny,bm,bn,split,a_pre,b_pre,out_f32" for kernel
// `id` into buf; returns -1 if id is out of range.
int aiter_amd_kernel_info(int id, char* buf, int buflen) {
    const Instance* in = find_by_id(id);
    if (!in || !buf || buflen <= 0) return -1;
    static const char* fam[] = {"a4w4", "a8w4", "a16w16"};
    snprintf(buf, buflen, "%d,%s,%s,%d,%d,%d,%d,%d,%d,%d", in->id, in->name.c_str(), fam[in->fam],
             (int)in->skinny, in->bm, in->bn, (int)in->split, (int)in->var.a_pre, (int)in->var.b_pre,
             (int)in->var.out_f32);
    return 0;
}

int aiter_amd_resolve_kernel_name(const char* name, int family, int a_pre, int b_pre, int out_f32, int64_t M) {
    if (!name || !name[0] || family < 0 || family > 2) return -2;
    bool known = false;
    const Instance* in = resolve_name(name, (Family)family, Variant{a_pre != 0, b_pre != 0, out_f32 != 0}, M, &known);
    return !known ? -2 : (in ? in->id : -1);
}

int aiter_amd_resolve_opus_kid(int kid, int out_f32, int64_t M) {
    RefTile t;
    if (!decode_opus_kid(kid, &t)) return -2;
    const Instance* in = reference_tile_instance(t, kA16W16, Variant{false, false, out_f32 != 0}, M);
    return in ? in->id : -1;
}

// fused_gemm_afp4wfp4_mul_add / fused_gemm_afp4wfp4_preshuffle_add_mul
// (aiter/ops/triton/gemm/fused/fused_gemm_afp4wfp4_mul_add.py:63-236, 239-...):
// out = a * (x w^T) + b (fuse_type 0) or a * b + x w^T (fuse_type 1), in f32,
// one rounding to bf16; a / b: tensors ([M, N], [1, N], [M, 1] or one element;
// f32 or bf16) or NULL for the scalar argument.
int fused_gemm_afp4wfp4_mul_add(aiter_tensor_t* x, aiter_tensor_t* w, aiter_tensor_t* x_scale, aiter_tensor_t* w_scale,
                                aiter_tensor_t* a, float a_scalar, aiter_tensor_t* b, float b_scalar, int fuse_type,
                                aiter_tensor_t* out, int preshuffled, const char* kernelName, aiter_stream_t stream) {
    return safe_call([&] {
        AA_CHECK(x && w && out, "x, w and out must be given");
        DeviceGuard g(x->device_id);
        AA_CHECK(fuse_type == 0 || fuse_type == 1, "fuse_type must be 0 or 1");
        AA_CHECK(out->dtype == AITER_DTYPE_bf16, "out must be bf16");
        const int64_t M = rows_2d(x), N = cols_2d(out);
        EpiOp e{};
        e.kind = 1;
        e.fuse = fuse_type;
        e.sa = a_scalar;
        e.sb = b_scalar;
        mul_add_operand(a, M, N, &e.ta, &e.ta_bf16, &e.ta_sm, &e.ta_sn, "a");
        mul_add_operand(b, M, N, &e.tb, &e.tb_bf16, &e.tb_sm, &e.tb_sn, "b");
        fused_a4w4(x, w, x_scale, w_scale, preshuffled != 0, out, nullptr, e, kernelName,
                   reinterpret_cast<hipStream_t>(stream));
    });
}

// fused_gemm_afp4wfp4_split_cat / fused_gemm_afp4wfp4_preshuffle_split_cat
// (aiter/ops/triton/gemm/fused/fused_gemm_afp4wfp4_split_cat.py:19-196, 199-...):
// C = x w^T viewed [M, D, S1+S2]; c1 = cat(C[..., :S1], y) [M, D, S1+S3],
// c2 = C[..., S1:] [M, D, S2]; bf16, c1 and c2 contiguous; S1, S2, S3
// multiples of 8 (whole 16-byte pieces per segment).
int fused_gemm_afp4wfp4_split_cat(aiter_tensor_t* x, aiter_tensor_t* w, aiter_tensor_t* x_scale,
                                  aiter_tensor_t* w_scale, aiter_tensor_t* y, aiter_tensor_t* c1, aiter_tensor_t* c2,
                                  int S1, int S2, int preshuffled, const char* kernelName, aiter_stream_t stream) {
    return safe_call([&] {
        AA_CHECK(x && w && y && c1 && c2, "x, w, y, c1 and c2 must be given");
        DeviceGuard g(x->device_id);
        check_tensor(y, "y", 3);
        AA_CHECK(y->ndim == 3 && y->dtype == AITER_DTYPE_bf16, "y must be [M, D, S3] bf16");
        const int64_t M = y->shape[0], D = y->shape[1], S3 = y->shape[2];
        AA_CHECK(rows_2d(x) == M, "x has ", rows_2d(x), " rows, y ", M);
        AA_CHECK(S1 > 0 && S2 > 0 && S1 % 8 == 0 && S2 % 8 == 0 && S3 % 8 == 0,
                 "S1, S2 and S3 must be positive multiples of 8 (got ", S1, ", ", S2, ", ", S3, ")");
        AA_CHECK(c1->dtype == AITER_DTYPE_bf16 && c2->dtype == AITER_DTYPE_bf16, "c1 and c2 must be bf16");
        const aiter_tensor_t c1v = flat_view(c1, M * D, S1 + S3, "c1");
        (void)flat_view(c2, M * D, S2, "c2");
        AA_CHECK(((uintptr_t)c1->ptr & 15) == 0 && ((uintptr_t)c2->ptr & 15) == 0, "c1 and c2 must be 16-byte aligned");
        const int64_t N = D * (S1 + S2);
        EpiOp e{};
        e.kind = 2;
        e.c2 = c2->ptr;
        e.s1 = S1;
        e.s2 = S2;
        e.s3 = (int)S3;
        e.ld1 = D * (S1 + S3);
        e.ld2 = D * S2;
        // the GEMM's own output descriptor: [M, N] at c1 (only its pointer is used)
        aiter_tensor_t outv = c1v;
        outv.ndim = 2;
        outv.shape[0] = M;
        outv.shape[1] = N;
        outv.strides[0] = N;
        outv.strides[1] = 1;
        outv.numel = (size_t)(M * N);
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        fused_a4w4(x, w, x_scale, w_scale, preshuffled != 0, &outv, nullptr, e, kernelName, st);
        const int64_t total = M * D * S3;
        if (total > 0) {
            split_cat_copy_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, st>>>(
                static_cast<const uint16_t*>(y->ptr), y->strides[0], y->strides[1], y->strides[2],
                static_cast<uint16_t*>(c1->ptr), (int)M, (int)D, S1, (int)S3);
            AA_HIP(hipGetLastError());
        }
    });
}

// fused_gemm_afp4wfp4_a16w16 (aiter/ops/triton/gemm/fused/fused_gemm_afp4wfp4_a16w16.py:23-254):
// y_fp4 = x_fp4 w_fp4^T (+ bias_fp4) and y_bf16 = x_bf16 w_bf16^T (+ bias_bf16)
// over the same M and K, bf16 out; biases f32 [N].  M <= 32 with no kernel
// named, and neither GEMM long enough in K for its skinny launch to split K:
// both GEMMs in one grid over both GEMMs' column blocks (skinny_pair_kernel,
// as the reference's one Triton grid of cdiv(N_fp4) + cdiv(N_bf16) tiles,
// :145-155); otherwise two launches (a split GEMM's workgroups would run its
// whole K inside the shared grid: measured 13.6 against 10.9 us at M = 1,
// 19.4 against 12.9 at M = 16 and 41.6 against 20.7 at M = 64 for
// N = 4096 + 256, K = 7168).
int fused_gemm_afp4wfp4_a16w16(aiter_tensor_t* x_fp4, aiter_tensor_t* w_fp4, aiter_tensor_t* x_fp4_scale,
                               aiter_tensor_t* w_fp4_scale, aiter_tensor_t* bias_fp4, aiter_tensor_t* y_fp4,
                               const char* kernel_fp4, aiter_tensor_t* x_bf16, aiter_tensor_t* w_bf16,
                               aiter_tensor_t* bias_bf16, aiter_tensor_t* y_bf16, const char* kernel_bf16,
                               int preshuffled, aiter_stream_t stream) {
    return safe_call([&] {
        AA_CHECK(x_fp4 && x_bf16, "x_fp4 and x_bf16 must be given");
        DeviceGuard g(x_fp4->device_id);
        check_tensor(x_fp4, "x_fp4", 2);
        check_tensor(x_bf16, "x_bf16", 2);
        AA_CHECK(rows_2d(x_fp4) == rows_2d(x_bf16), "x_fp4 and x_bf16 must have the same M");
        AA_CHECK(cols_2d(x_fp4) * 2 == cols_2d(x_bf16), "x_fp4 and x_bf16 must have the same K");
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        const int64_t M = rows_2d(x_fp4);
        const bool named = (kernel_fp4 && kernel_fp4[0]) || (kernel_bf16 && kernel_bf16[0]);
        bool one_grid = M > 0 && M <= 32 && !named;
        if (one_grid) {
            int dev = x_fp4->device_id;
            if (dev < 0) AA_HIP(hipGetDevice(&dev));
            const int cus = device_cu_count(dev);
            const int64_t K = cols_2d(x_bf16);
            check_tensor(w_fp4, "w_fp4", 2);
            check_tensor(w_bf16, "w_bf16", 2);
            const int n4 = (int)rows_2d(w_fp4), n16 = (int)rows_2d(w_bf16);
            one_grid = skinny_splits((n4 + 15) / 16, (int)(K / 128), cus) == 1 &&
                       skinny_splits((n16 + 15) / 16, (int)(K / 32), cus) == 1;
        }
        if (one_grid) {
            const int mf = M <= 16 ? 1 : 2;
            const std::string n4 = "a4w4_skinny_m" + std::to_string(16 * mf) + (preshuffled ? "" : "_bplain");
            const std::string n16 = "a16w16_skinny_m" + std::to_string(16 * mf) + "_bplain";
            GemmParams pa{}, pb{};
            fused_a4w4(x_fp4, w_fp4, x_fp4_scale, w_fp4_scale, preshuffled != 0, y_fp4, bias_fp4, EpiOp{},
                       n4.c_str(), st, &pa);
            GemmCall c{kA16W16, {false, false, false}, x_bf16, w_bf16, nullptr, nullptr, y_bf16, bias_bf16,
                       1.0f, 1.0f, n16.c_str(), -1, -1};
            c.capture = &pb;
            run_gemm(c, st);
            const int nblk_a = (pa.N + 15) / 16, nblk_b = (pb.N + 15) / 16;
            if (nblk_a + nblk_b == 0) return;
            const dim3 grid((unsigned)(nblk_a + nblk_b));
#define AA_PAIR(MF)                                                                               \
    (preshuffled ? skinny_pair_kernel<MF, true><<<grid, 512, 0, st>>>(pa, pb, nblk_a)             \
                 : skinny_pair_kernel<MF, false><<<grid, 512, 0, st>>>(pa, pb, nblk_a))
            if (mf == 1) AA_PAIR(1);
            else AA_PAIR(2);
#undef AA_PAIR
            AA_HIP(hipGetLastError());
            return;
        }
        fused_a4w4(x_fp4, w_fp4, x_fp4_scale, w_fp4_scale, preshuffled != 0, y_fp4, bias_fp4, EpiOp{}, kernel_fp4, st);
        GemmCall c{kA16W16, {false, false, false}, x_bf16, w_bf16, nullptr, nullptr, y_bf16, bias_bf16,
                   1.0f, 1.0f, kernel_bf16, -1, -1};
        run_gemm(c, st);
    });
}

// Bytes of the split-K workspace held for (device, stream), 0 if none
// (introspection: the tests read what a call reserved).
int64_t aiter_amd_workspace_bytes(int device, aiter_stream_t stream) {
    std::lock_guard<std::mutex> lk(workspace_mutex());
    auto& ws = workspace_map();
    auto it = ws.find(WsKey{device, reinterpret_cast<hipStream_t>(stream), 0});
    return it == ws.end() ? 0 : (int64_t)it->second.bytes;
}

// Frees every library workspace held for (device, stream) after the
// stream's work completes; the next call that needs one allocates it again.
int aiter_amd_workspace_release(int device, aiter_stream_t stream) {
    return safe_call([&] {
        DeviceGuard g(device);
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        AA_HIP(hipStreamIsCapturing(st, &cs));
        AA_CHECK(cs == hipStreamCaptureStatusNone, "workspaces cannot be released during graph capture");
        std::lock_guard<std::mutex> lk(workspace_mutex());
        auto& ws = workspace_map();
        for (auto it = ws.begin(); it != ws.end();) {
            if (it->first.dev == device && it->first.st == st) {
                if (it->second.ptr) {
                    AA_HIP(hipStreamSynchronize(st));
                    AA_HIP(hipFree(it->second.ptr));
                }
                it = ws.erase(it);
            } else {
                ++it;
            }
        }
    });
}

// Pre-size the split-K workspace of (device, stream) before graph capture.
int gemm_workspace_reserve(int device, aiter_stream_t stream, size_t bytes) {
    return safe_call([&] {
        DeviceGuard g(device);
        (void)workspace(device, reinterpret_cast<hipStream_t>(stream), bytes);
        (void)lib_counters(device, reinterpret_cast<hipStream_t>(stream), 0);   // the split-K tile counters
    });
}

}  // extern "C"
