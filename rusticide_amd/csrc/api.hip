// api.hip -- the C ABI of include/rusticide_hip.h.
//
// Host-side mirror of rusticide's kernel facade for the quantized path:
// Matrix::load_on (crates/rusticide-model/src/weights.rs:53-98) becomes a
// one-time upload to HBM, and matmul_batch
// (crates/rusticide-kernels/src/matmul.rs:229-248) becomes: quantize each
// activation kind once per batch on the device, then one grouped GEMV launch
// per weight format covering every matrix of that format.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/rusticide_hip.h"
#include "rh_internal.h"

using namespace rh;

struct rh_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string last_error;
  // scratch, grown on demand
  void* buf[9] = {};
  size_t cap[9] = {};
  Q8Dev super_q, row_q;
  // bumped whenever a scratch slot moves: graphs that captured the old
  // addresses must not be replayed
  uint64_t scratch_gen = 0;
  // the split GEMMs' tile arrival counters (kFixupTiles, zero between
  // launches); nullptr: every split GEMM combines in a launch of its own
  uint32_t* tile_counters = nullptr;
  // pinned staging for matrix uploads, made on the first one
  uint8_t* stage[2] = {};
  hipEvent_t stage_done[2] = {};
};

struct rh_matrix {
  rh_ctx* ctx = nullptr;
  int device = 0;  // freeing needs no live context
  uint32_t type_id = 0;
  size_t rows = 0, cols = 0;
  size_t row_bytes = 0;  // bytes of one row's data (f32 for dense)
  size_t stride = 0;     // bytes between rows in HBM
  size_t nblocks = 0;    // blocks per row (elements for dense)
  float scale = 0.0f;
  uint8_t* data = nullptr;
  size_t bytes = 0;
};

struct rh_q8 {
  rh_ctx* ctx = nullptr;
  int device = 0;
  int kind = 0;
  size_t width = 0, tokens = 0;
  Q8Dev q;
  void* mem = nullptr;
  size_t cap = 0;
};

namespace {

enum Scratch { kIn = 0, kOut, kQuants, kScales, kSums, kSums16, kRaw, kRowQ, kTerms, kScratchSlots };
static_assert(kScratchSlots == sizeof(rh_ctx::cap) / sizeof(size_t), "one scratch slot per Scratch value");

// Batches of this many tokens or more run Q4_K, Q6_K and I2_S on the MFMA GEMMs.
size_t g_gemm_min_tokens = 9;

rh_status fail(rh_ctx* ctx, rh_status st, const std::string& msg) {
  if (ctx) ctx->last_error = msg;
  return st;
}

rh_status hip_fail(rh_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, e == hipErrorOutOfMemory ? RH_ERR_OUT_OF_MEMORY : RH_ERR_DEVICE,
              std::string(what) + ": " + hipGetErrorString(e));
}

#define RH_HIP(ctx, expr)                            \
  do {                                               \
    hipError_t e_ = (expr);                          \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, #expr); \
  } while (0)

size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

// Which GEMV kernel family serves a format (Tuning::gemv). The default is
// one launch per format in which the kernels quantize the activation
// themselves (decode-sized batches; larger ones fall back to a quantize
// launch plus kernels that read its result, the kLds family).
enum class Family { kFused, kLds };

Family family() { return tuning().gemv == 1 ? Family::kLds : Family::kFused; }

unsigned format_bit(uint32_t type_id) {
  return type_id == RH_TYPE_Q4_K ? 1u : type_id == RH_TYPE_Q6_K ? 2u : type_id == RH_TYPE_I2_S ? 4u : 0u;
}

// Grows scratch slot `i` to at least `bytes`.
rh_status ensure(rh_ctx* ctx, int i, size_t bytes) {
  if (ctx->cap[i] >= bytes) return RH_OK;
  if (ctx->buf[i]) {
    // work queued on any stream may still read the old buffer
    RH_HIP(ctx, hipDeviceSynchronize());
    RH_HIP(ctx, hipFree(ctx->buf[i]));
    ctx->buf[i] = nullptr;
    ctx->cap[i] = 0;
  }
  size_t want = round_up(bytes < 4096 ? 4096 : bytes, 4096);
  ctx->scratch_gen++;
  RH_HIP(ctx, hipMalloc(&ctx->buf[i], want));
  ctx->cap[i] = want;
  return RH_OK;
}

bool is_kquant(uint32_t t) { return t == RH_TYPE_Q4_K || t == RH_TYPE_Q6_K; }

// Block geometry (quantize/src/format.rs:31-92).
bool geometry(uint32_t type_id, size_t* bs, size_t* bb) {
  switch (type_id) {
    case RH_TYPE_Q4_K: *bs = 256; *bb = 144; return true;
    case RH_TYPE_Q6_K: *bs = 256; *bb = 210; return true;
    case RH_TYPE_I2_S: *bs = 128; *bb = 32; return true;
    default: return false;
  }
}

// Activation buffers for `tokens` rows of `width` values, both kinds.
rh_status ensure_q8(rh_ctx* ctx, size_t width, size_t tokens) {
  const size_t qstride = round_up(width < 256 ? 256 : width, 256);
  const size_t bstride = round_up(qstride / 32, 8);
  rh_status st;
  if ((st = ensure(ctx, kQuants, 2 * tokens * qstride)) != RH_OK) return st;
  if ((st = ensure(ctx, kScales, 2 * tokens * bstride * sizeof(float))) != RH_OK) return st;
  if ((st = ensure(ctx, kSums, 2 * tokens * bstride * sizeof(int32_t))) != RH_OK) return st;
  if ((st = ensure(ctx, kSums16, 3 * tokens * bstride * sizeof(int32_t))) != RH_OK) return st;
  Q8Dev s;
  s.qstride = qstride;
  s.bstride = bstride;
  s.quants = static_cast<int8_t*>(ctx->buf[kQuants]);
  s.scales = static_cast<float*>(ctx->buf[kScales]);
  s.sums = static_cast<int32_t*>(ctx->buf[kSums]);
  s.sums16 = static_cast<int32_t*>(ctx->buf[kSums16]);
  s.n_blocks = width / 256 * 8;
  Q8Dev r = s;
  r.quants = s.quants + tokens * qstride;
  r.scales = s.scales + tokens * bstride;
  r.sums = s.sums + tokens * bstride;
  r.sums16 = s.sums16 + 2 * tokens * bstride;  // per-16 sums: super kind only
  r.n_blocks = width / 32;
  ctx->super_q = s;
  ctx->row_q = r;
  return RH_OK;
}

// Rows worth computing: out_len bounds them (quant_kernel.rs:106-111).
size_t rows_for(const rh_matrix* m, size_t out_len, size_t tokens) {
  size_t by_out = (out_len + tokens - 1) / tokens;
  return m->rows < by_out ? m->rows : by_out;
}

// One grouped launch per format over `jobs`, against quantized activations
// `super_q` / `row_q` (or the raw f32 inputs for dense rows).
// `fused` holds, per format (bit 0 Q4_K, 1 Q6_K, 2 I2_S), whether its
// launches quantize d_in themselves.
rh_status launch_jobs(rh_ctx* ctx, const float* d_in, size_t width, size_t tokens, const rh_job* jobs,
                      size_t n_jobs, const Q8Dev& super_q, const Q8Dev& row_q, hipStream_t s,
                      int32_t* raw, unsigned fused, bool allow_split = true, bool token_major = false,
                      SplitOut* defer = nullptr) {
  rh_status st = RH_OK;
  const uint32_t kinds[4] = {RH_TYPE_Q4_K, RH_TYPE_Q6_K, RH_TYPE_I2_S, RH_TYPE_F32};
  for (uint32_t kind : kinds) {
    GemvJobs g{};
    uint32_t nbmax = 0;
    auto flush = [&]() -> rh_status {
      if (g.n == 0) return RH_OK;
      const Q8Dev& q = kind == RH_TYPE_I2_S ? row_q : super_q;
      if (is_kquant(kind) && tokens >= g_gemm_min_tokens) {
        if (!gemm_fits(tokens, q.qstride))
          return fail(ctx, RH_ERR_INVALID_ARGUMENT, "a batch's quantized activation exceeds 4 GiB");
        float* terms = nullptr;  // without it the GEMM runs unsplit (the same bits)
        if (const size_t tb = allow_split ? gemm_split_bytes(kind, g, tokens) : 0) {
          rh_status es = ensure(ctx, kTerms, tb);
          if (es != RH_OK) return es;
          terms = static_cast<float*>(ctx->buf[kTerms]);
        }
        RH_HIP(ctx, launch_gemm(kind, g, q, tokens, terms, s, defer, ctx->tile_counters));
        g = GemvJobs{};
        nbmax = 0;
        return RH_OK;
      }
      if (kind == RH_TYPE_I2_S && tokens >= g_gemm_min_tokens) {
        RH_HIP(ctx, launch_gemm_i2s(g, q, tokens, raw, s));
        g = GemvJobs{};
        nbmax = 0;
        return RH_OK;
      }
      size_t tmax = kMaxTokens;
      if (kind != RH_TYPE_F32) tmax = gemv_max_tokens(kind, nbmax);
      if (tmax == 0) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "rows too wide for the GEMV kernels");
      if (fused & format_bit(kind)) {
        RH_HIP(ctx, launch_gemv_fused(kind, g, d_in, width, tokens, 0, tokens, s, raw));
        g = GemvJobs{};
        nbmax = 0;
        return RH_OK;
      }
      for (size_t t0 = 0; t0 < tokens; t0 += tmax) {
        size_t tn = tokens - t0 < tmax ? tokens - t0 : tmax;
        RH_HIP(ctx, launch_gemv(kind, g, q, d_in, width, tokens, t0, tn, s, raw));
      }
      g = GemvJobs{};
      nbmax = 0;
      return RH_OK;
    };
    for (size_t i = 0; i < n_jobs; i++) {
      const rh_matrix* m = jobs[i].weights;
      const uint32_t t = (m->type_id == RH_TYPE_F16) ? RH_TYPE_F32 : m->type_id;
      if (t != kind) continue;
      const size_t rows = rows_for(m, jobs[i].out_len, tokens);
      if (rows == 0) continue;
      size_t nb;
      if (kind == RH_TYPE_F32) nb = m->cols < width ? m->cols : width;
      else if (kind == RH_TYPE_I2_S) nb = row_q.n_blocks / 4;
      else nb = super_q.n_blocks / 8;
      if (kind != RH_TYPE_F32 && m->nblocks < nb) nb = m->nblocks;
      GemvJob& j = g.j[g.n++];
      j.w = m->data;
      j.ub = static_cast<uint32_t>(m->nblocks);
      j.stride = static_cast<uint32_t>(m->stride);
      j.rows = static_cast<uint32_t>(rows);
      j.nb = static_cast<uint32_t>(nb);
      j.out = jobs[i].out;
      j.out_len = jobs[i].out_len;
      j.scale = m->scale;
      j.tmajor = token_major ? 1u : 0u;
      if (kind != RH_TYPE_F32 && nb > nbmax) nbmax = static_cast<uint32_t>(nb);
      if (g.n == static_cast<uint32_t>(kMaxJobs) && (st = flush()) != RH_OK) return st;
    }
    if ((st = flush()) != RH_OK) return st;
  }
  return RH_OK;
}

// With `fixed`, the quantized activations go to the two Q8Dev of `fixed`
// (super-block, row kind) and nothing is allocated: the context's scratch is
// not grown and the GEMMs do not split K.
rh_status run_batch(rh_ctx* ctx, const float* d_in, size_t inputs_len, size_t tokens,
                    const rh_job* jobs, size_t n_jobs, hipStream_t s, int32_t* raw,
                    const Q8Dev* fixed = nullptr) {
  const size_t width = inputs_len / tokens;
  uint32_t nbmax[3] = {0, 0, 0};  // Q4_K, Q6_K, I2_S
  for (size_t i = 0; i < n_jobs; i++) {
    if (!jobs[i].weights) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "a job has no matrix");
    if (!jobs[i].out && jobs[i].out_len) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "a job has no output");
    const rh_matrix* m = jobs[i].weights;
    const unsigned bit = format_bit(m->type_id);
    if (!bit) continue;
    const size_t cover = m->type_id == RH_TYPE_I2_S ? width / 128 : width / 256;
    const uint32_t nb = static_cast<uint32_t>(m->nblocks < cover ? m->nblocks : cover);
    uint32_t& n = nbmax[bit >> 1];
    n = nb > n ? nb : n;
  }
  // A format is fused when its family allows it and the batch fits one
  // fused launch; otherwise its activation is quantized once here.
  unsigned present = 0, fused = 0;
  for (size_t i = 0; i < n_jobs; i++) present |= format_bit(jobs[i].weights->type_id);
  const uint32_t kinds[3] = {RH_TYPE_Q4_K, RH_TYPE_Q6_K, RH_TYPE_I2_S};
  for (int k = 0; k < 3; k++) {
    const uint32_t kind = kinds[k];
    const unsigned bit = format_bit(kind);
    if (!(present & bit) || family() != Family::kFused || !gemv_fused_ok(kind, width, tokens)) continue;
    if (kind != RH_TYPE_I2_S && tokens >= g_gemm_min_tokens) continue;
    if (tokens > gemv_max_tokens(kind, nbmax[bit >> 1])) continue;
    fused |= bit;
  }
  const bool need_super = (present & ~fused & 3u) != 0;
  const bool need_row = (present & ~fused & 4u) != 0;
  if (!fixed) {
    rh_status st = ensure_q8(ctx, width, tokens);
    if (st != RH_OK) return st;
  }
  const Q8Dev& sq = fixed ? fixed[0] : ctx->super_q;
  const Q8Dev& rq = fixed ? fixed[1] : ctx->row_q;
  if (need_super) RH_HIP(ctx, launch_quantize_super(d_in, width, tokens, sq, s));
  if (need_row) RH_HIP(ctx, launch_quantize_row(d_in, width, tokens, rq, s));
  return launch_jobs(ctx, d_in, width, tokens, jobs, n_jobs, sq, rq, s, raw, fused, fixed == nullptr);
}

// The allocation-free entry point's device memory: the quantized
// activations of one batch, both kinds, in a file-scope array of every GPU
// the library runs on. Host code reaches it only through the address
// hipGetSymbolAddress gives on each device (scratch_setup), never by name.
constexpr size_t kScratchBytes = RH_NOALLOC_SCRATCH_BYTES;
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

// The bytes of the activation layout q8_layout builds for `tokens` rows of
// `width` values (each part 256-byte aligned).
size_t q8_layout_bytes(size_t width, size_t tokens) {
  const size_t qstride = round_up(width < 256 ? 256 : width, 256);
  const size_t bstride = round_up(qstride / 32, 8);
  return 2 * round_up(tokens * qstride, 256) + 6 * round_up(tokens * bstride * 4, 256);
}

// Both activation kinds of a batch laid out from `base`: quants, scales,
// per-32 sums and (super-block kind) per-16 sums, as ensure_q8 lays them out
// in the context's buffers.
void q8_layout(uint8_t* base, size_t width, size_t tokens, Q8Dev out[2]) {
  const size_t qstride = round_up(width < 256 ? 256 : width, 256);
  const size_t bstride = round_up(qstride / 32, 8);
  const size_t qb = round_up(tokens * qstride, 256), fb = round_up(tokens * bstride * 4, 256);
  for (int k = 0; k < 2; k++) {
    Q8Dev& q = out[k];
    q.qstride = qstride;
    q.bstride = bstride;
    q.quants = reinterpret_cast<int8_t*>(base + k * qb);
    q.scales = reinterpret_cast<float*>(base + 2 * qb + k * fb);
    q.sums = reinterpret_cast<int32_t*>(base + 2 * qb + (2 + k) * fb);
    q.sums16 = reinterpret_cast<int32_t*>(base + 2 * qb + 4 * fb);  // two per 32-block, super-block kind
    q.n_blocks = k == 0 ? width / 256 * 8 : width / 32;
  }
}
}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
// Finds the array's address on `device` (current) once per process.
hipError_t scratch_setup(int device) {
  if (device < 0 || device >= kScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return hipSuccess;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e == hipSuccess) g_scratch_ptr[device] = ptr;
  return e;
}

void* scratch_ptr(int device) {
  if (device < 0 || device >= kScratchDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch_ptr[device];
}

}  // namespace

namespace rh {

int device_cus() {
  static const int cus = [] {
    int dev = 0, n = 0;
    return hipGetDevice(&dev) == hipSuccess &&
                   hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
               ? n
               : 256;
  }();
  return cus;
}

namespace {
// The current snapshot. A reload publishes a new one and never frees the
// old: a launch on another thread may still be reading it (a few dozen bytes
// per rh_reload_tuning call).
const Tuning g_default_tuning{};
std::atomic<const Tuning*> g_tuning{&g_default_tuning};
std::once_flag g_tuning_once;

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}
}  // namespace

const Tuning& tuning() { return *g_tuning.load(std::memory_order_acquire); }

void load_tuning() {
  Tuning t;
  if (const char* v = std::getenv("RUSTICIDE_HIP_GEMV")) {
    if (std::strcmp(v, "lds") == 0) t.gemv = 1;
  }
  const int ni = env_int("RUSTICIDE_HIP_GEMV_NI", 0);
  t.gemv_ni = ni == 1 || ni == 2 || ni == 4 || ni == 8 ? ni : 0;
  t.interleave = env_int("RUSTICIDE_HIP_GEMV_IL", 1) != 0;
  const int nni = env_int("RUSTICIDE_HIP_NORM_NI", 0);
  t.norm_ni = nni == 2 || nni == 4 ? nni : 0;
  const int knt = env_int("RUSTICIDE_HIP_KQ_NT", 0);
  t.kq_nt = knt == 256 || knt == 512 ? knt : 0;
  const int nnt = env_int("RUSTICIDE_HIP_NORM_NT", 0);
  t.norm_nt = nnt == 256 || nnt == 512 ? nnt : 0;
  t.kq_fix = env_int("RUSTICIDE_HIP_KQ_FIX", 1) != 0;
  t.kq_balance = env_int("RUSTICIDE_HIP_KQ_BALANCE", 1) != 0;
  t.kq_onepass = env_int("RUSTICIDE_HIP_KQ_ONEPASS", 1) != 0;
  const int gr = env_int("RUSTICIDE_HIP_I2S_GROUPS", 0);
  t.i2s_groups = gr == 1 || gr == 2 || gr == 4 ? gr : 0;
  const int lpr = env_int("RUSTICIDE_HIP_I2S_LPR", 0);
  t.i2s_lpr = lpr == 8 || lpr == 16 || lpr == 32 || lpr == 64 ? lpr : 0;
  t.i2s_one = env_int("RUSTICIDE_HIP_I2S_ONE", 1) != 0;
  const int nt = env_int("RUSTICIDE_HIP_I2S_NT", 0);
  t.i2s_nt = nt == 256 || nt == 512 || nt == 1024 ? nt : 0;
  const int bn = env_int("RUSTICIDE_HIP_GEMM_BN", 0);
  t.gemm_bn = bn == 32 || bn == 64 ? bn : 0;
  t.gemm_split = env_int("RUSTICIDE_HIP_GEMM_SPLIT", 1) != 0;
  t.gemm_fixup = env_int("RUSTICIDE_HIP_GEMM_FIXUP", 1) != 0;
  t.attn_lds = env_int("RUSTICIDE_HIP_ATTN_LDS", 1) != 0;
  g_tuning.store(new Tuning(t), std::memory_order_release);
}

void init_tuning() { std::call_once(g_tuning_once, load_tuning); }

int ctx_device(const rh_ctx* ctx) { return ctx->device; }
uint64_t ctx_scratch_generation(const rh_ctx* ctx) { return ctx->scratch_gen; }

rh_status matmul_norm_device(rh_ctx* ctx, const float* hidden, const NormIn& norm, size_t width, const rh_job* jobs,
                             size_t n_jobs, hipStream_t s) {
  if (!ctx || !hidden || !norm.weight || !jobs || n_jobs == 0) return RH_ERR_INVALID_ARGUMENT;
  for (size_t i = 0; i < n_jobs; i++)
    if (!jobs[i].weights || !is_kquant(jobs[i].weights->type_id) || (!jobs[i].out && jobs[i].out_len))
      return fail(ctx, RH_ERR_INVALID_ARGUMENT, "a norm-fused job is not a k-quant matrix with an output");
  for (uint32_t kind : {static_cast<uint32_t>(RH_TYPE_Q4_K), static_cast<uint32_t>(RH_TYPE_Q6_K)}) {
    GemvJobs g{};
    for (size_t i = 0; i < n_jobs; i++) {
      const rh_matrix* m = jobs[i].weights;
      if (m->type_id != kind) continue;
      const size_t rows = rows_for(m, jobs[i].out_len, 1);
      if (rows == 0) continue;
      if (g.n == static_cast<uint32_t>(kMaxJobs)) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "too many jobs");
      const size_t cover = width / 256;
      GemvJob& j = g.j[g.n++];
      j.w = m->data;
      j.stride = static_cast<uint32_t>(m->stride);
      j.rows = static_cast<uint32_t>(rows);
      j.nb = static_cast<uint32_t>(m->nblocks < cover ? m->nblocks : cover);
      j.ub = static_cast<uint32_t>(m->nblocks);
      j.out = jobs[i].out;
      j.out_len = jobs[i].out_len;
      j.scale = m->scale;
    }
    if (g.n) RH_HIP(ctx, launch_gemv_fused(kind, g, hidden, width, 1, 0, 1, s, nullptr, &norm));
  }
  return RH_OK;
}
bool gate_up_pairable(const rh_matrix* gate, const rh_matrix* up, size_t width) {
  return gate && up && is_kquant(gate->type_id) && gate->type_id == up->type_id && gate->cols == width &&
         up->cols == width && gate->rows == up->rows && gate->stride == up->stride &&
         gate->nblocks == up->nblocks && gate->nblocks == width / 256 &&
         norm_fusable(gate->type_id, width, static_cast<uint32_t>(width / 256));
}

rh_status matmul_norm_silu_device(rh_ctx* ctx, const float* hidden, const NormIn& norm, size_t width,
                                  const rh_matrix* gate, const rh_matrix* up, float* out, size_t rows, hipStream_t s) {
  if (!ctx || !hidden || !norm.weight || !out) return RH_ERR_INVALID_ARGUMENT;
  if (!gate_up_pairable(gate, up, width) || rows > gate->rows)
    return fail(ctx, RH_ERR_INVALID_ARGUMENT, "gate and up are not one k-quant shape");
  if (rows == 0) return RH_OK;
  GemvJobs g{};
  GemvJob& j = g.j[g.n++];
  j.w = gate->data;
  j.w2 = up->data;
  j.ub = static_cast<uint32_t>(gate->nblocks);
  j.stride = static_cast<uint32_t>(gate->stride);
  j.rows = static_cast<uint32_t>(rows);
  j.nb = static_cast<uint32_t>(gate->nblocks);
  j.out = out;
  j.out_len = rows;
  j.scale = gate->scale;
  RH_HIP(ctx, launch_gemv_fused(gate->type_id, g, hidden, width, 1, 0, 1, s, nullptr, &norm));
  return RH_OK;
}

rh_status matmul_q8_device(rh_ctx* ctx, const Q8Dev& q, size_t width, size_t tokens, const rh_job* jobs,
                           size_t n_jobs, hipStream_t s, bool token_major, SplitOut* defer) {
  if (!ctx || (!jobs && n_jobs) || tokens == 0) return RH_ERR_INVALID_ARGUMENT;
  if (defer && (!token_major || n_jobs != 1)) return RH_ERR_INVALID_ARGUMENT;
  if (defer) *defer = SplitOut{};
  for (size_t i = 0; i < n_jobs; i++)
    if (!jobs[i].weights || !is_kquant(jobs[i].weights->type_id) || (!jobs[i].out && jobs[i].out_len))
      return fail(ctx, RH_ERR_INVALID_ARGUMENT, "a pre-quantized job is not a k-quant matrix with an output");
  if (token_major && tokens < g_gemm_min_tokens)
    return fail(ctx, RH_ERR_INVALID_ARGUMENT, "token-major outputs need the GEMM path's token count");
  return launch_jobs(ctx, nullptr, width, tokens, jobs, n_jobs, q, q, s, nullptr, 0u, true, token_major, defer);
}

// Calls made without a context keep their message per thread
// (rh_last_error(NULL)).
thread_local std::string t_last_error;

rh_status set_last_error(rh_ctx* ctx, rh_status st, const std::string& msg) {
  if (ctx) return fail(ctx, st, msg);
  t_last_error = msg;
  return st;
}

const uint8_t* matrix_data(const rh_matrix* m) { return m->data; }
size_t matrix_pitch(const rh_matrix* m) { return is_kquant(m->type_id) ? m->nblocks : m->stride; }

rh_status matrix_prepare(rh_ctx* ctx, uint32_t type_id, const void* data, size_t len, size_t rows, size_t cols,
                         PendingUpload* out) {
  if (!ctx || !out || (!data && len)) return RH_ERR_INVALID_ARGUMENT;
  out->m = nullptr;
  if (cols == 0) return fail(ctx, RH_ERR_INVALID_CONFIG, "a weight matrix has no columns");
  RH_HIP(ctx, hipSetDevice(ctx->device));
  rh_matrix* m = new (std::nothrow) rh_matrix();
  if (!m) return fail(ctx, RH_ERR_OUT_OF_MEMORY, "host allocation failed");
  m->ctx = ctx;
  m->device = ctx->device;
  m->type_id = type_id;
  m->rows = rows;
  m->cols = cols;
  const uint8_t* src = static_cast<const uint8_t*>(data);
  size_t bs = 0, bb = 0;
  if (type_id == RH_TYPE_F32 || type_id == RH_TYPE_F16) {
    const size_t esz = type_id == RH_TYPE_F32 ? 4 : 2;
    if (rows && len / esz / rows < cols) {
      delete m;
      return fail(ctx, RH_ERR_SHAPE_MISMATCH, "data too short for rows x cols");
    }
    if (type_id == RH_TYPE_F16) {  // widen (model/src/weights.rs:241-247)
      try {
        out->widened.resize(rows * cols);
      } catch (const std::bad_alloc&) {
        delete m;
        return fail(ctx, RH_ERR_OUT_OF_MEMORY, "host allocation failed");
      }
      for (size_t i = 0; i < rows * cols; i++) {
        _Float16 f;
        std::memcpy(&f, src + 2 * i, 2);
        out->widened[i] = static_cast<float>(f);
      }
      src = reinterpret_cast<const uint8_t*>(out->widened.data());
      m->type_id = RH_TYPE_F32;
    }
    m->row_bytes = cols * 4;
    m->stride = m->row_bytes;
    m->nblocks = cols;
    // the GEMV jobs carry a row count and a row stride in 32 bits
    if (rows > size_t{0xffffffffu} || m->stride > size_t{0xffffffffu}) {
      delete m;
      return fail(ctx, RH_ERR_SHAPE_MISMATCH, "dense matrix exceeds 2^32 rows or 4 GiB per row");
    }
  } else if (geometry(type_id, &bs, &bb)) {
    if (cols % bs != 0) {
      delete m;
      return fail(ctx, RH_ERR_SHAPE_MISMATCH, "cols is not a whole number of blocks");
    }
    m->nblocks = cols / bs;
    m->row_bytes = m->nblocks * bb;
    m->stride = round_up(m->row_bytes, 16);
    // the GEMV kernels address a matrix with 24-bit row indices and 32-bit
    // byte offsets
    if (rows >= (size_t{1} << 24) || m->stride >= (size_t{1} << 24) ||
        rows * m->stride + kPad > size_t{0xffffffffu} ||
        (is_kquant(type_id) && units_bytes(type_id, rows, m->nblocks) + kPad > size_t{0xffffffffu})) {
      delete m;
      return fail(ctx, RH_ERR_SHAPE_MISMATCH, "matrix exceeds 2^24 rows or 4 GiB of blocks");
    }
    const size_t body = rows * m->row_bytes;
    if (type_id == RH_TYPE_I2_S) {
      // model/src/weights.rs:70-80,190-202: the trailer's leading f32
      if (len < body || len - body < 4) {
        delete m;
        return fail(ctx, RH_ERR_INVALID_TENSOR, "its data is too short to hold its scale");
      }
      float scale;
      std::memcpy(&scale, src + body, 4);
      if (!std::isfinite(scale)) {
        delete m;
        return fail(ctx, RH_ERR_INVALID_TENSOR, "its scale is not finite");
      }
      m->scale = scale;
    } else if (len < body) {
      delete m;
      return fail(ctx, RH_ERR_SHAPE_MISMATCH, "data too short for rows x cols");
    }
  } else {
    delete m;
    return fail(ctx, RH_ERR_MISSING_KERNEL, "no kernel reads this block format");
  }
  // Q4_K / Q6_K live in the unit layout (rh_device.h), whole groups of 16
  // blocks; I2_S and dense rows at the 16-byte stride. kPad bytes of zeros
  // follow either.
  m->bytes = round_up((is_kquant(type_id) ? units_bytes(type_id, rows, m->nblocks) : rows * m->stride) + kPad, 256);
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&m->data), m->bytes);
  if (e != hipSuccess) {
    delete m;
    return hip_fail(ctx, e, "hipMalloc(matrix)");
  }
  out->m = m;
  out->src = src;
  return RH_OK;
}

namespace {

constexpr size_t kStageBytes = size_t{32} << 20;  // per pinned staging buffer
constexpr size_t kCopySlice = size_t{2} << 20;    // least bytes one host thread copies

// Group g of a k-quant matrix in the unit layout (rh_device.h) into dst,
// from its blocks back to back in src (blocks past the last are zeros).
void unit_group_image(const rh_matrix* m, const uint8_t* src, size_t g, uint8_t* dst) {
  const size_t total = m->rows * m->nblocks;
  if (m->type_id == RH_TYPE_Q4_K) {
    for (size_t tw = 0; tw < 16; tw++) {
      const size_t e = 16 * g + tw;
      if (e >= total) {
        std::memset(dst + 16 * tw, 0, 16);
        std::memset(dst + 256 + 64 * tw, 0, 64);
        std::memset(dst + 1280 + 64 * tw, 0, 64);
        continue;
      }
      const uint8_t* b = src + e * 144;
      std::memcpy(dst + 16 * tw, b, 16);
      std::memcpy(dst + 256 + 64 * tw, b + 16, 64);
      std::memcpy(dst + 1280 + 64 * tw, b + 80, 64);
    }
    return;
  }
  for (size_t tw = 0; tw < 16; tw++) {
    const size_t e = 16 * g + tw;
    uint8_t zero[210] = {};
    const uint8_t* b = e < total ? src + e * 210 : zero;
    for (size_t h = 0; h < 2; h++) {
      std::memcpy(dst + 64 * tw + 32 * h, b + 64 * h, 32);
      std::memcpy(dst + 1024 + 64 * tw + 32 * h, b + 64 * h + 32, 32);
    }
    std::memcpy(dst + 2048 + 64 * tw, b + 128, 64);
    std::memcpy(dst + 3072 + 16 * tw, b + 192, 16);
    std::memcpy(dst + 3328 + 2 * tw, b + 208, 2);
  }
}

// Bytes [lo, hi) of a matrix's device image: for Q4_K / Q6_K the unit
// layout, for I2_S and dense rows row r's data at r * stride; zeros in the
// gaps between rows and after the last one.
void image_range(const rh_matrix* m, const uint8_t* src, size_t lo, size_t hi, uint8_t* dst) {
  if (is_kquant(m->type_id)) {
    const size_t gb = m->type_id == RH_TYPE_Q4_K ? 16 * 144 : 16 * 210;
    const size_t body = units_bytes(m->type_id, m->rows, m->nblocks);
    uint8_t tmp[16 * 210];
    for (size_t pos = lo; pos < hi;) {
      if (pos >= body) {
        std::memset(dst + (pos - lo), 0, hi - pos);
        return;
      }
      const size_t g = pos / gb, in = pos - g * gb, take = std::min(hi - pos, gb - in);
      if (in == 0 && take == gb) {
        unit_group_image(m, src, g, dst + (pos - lo));
      } else {  // a group cut by the range: build it whole, copy the part
        unit_group_image(m, src, g, tmp);
        std::memcpy(dst + (pos - lo), tmp + in, take);
      }
      pos += take;
    }
    return;
  }
  const size_t body = m->rows * m->stride;
  size_t pos = lo;
  while (pos < hi) {
    if (pos >= body) {
      std::memset(dst + (pos - lo), 0, hi - pos);
      return;
    }
    if (m->stride == m->row_bytes) {  // rows back to back: one copy
      const size_t e = hi < body ? hi : body;
      std::memcpy(dst + (pos - lo), src + pos, e - pos);
      pos = e;
      continue;
    }
    const size_t r = pos / m->stride, in = pos - r * m->stride;
    const size_t end = std::min(hi, (r + 1) * m->stride);
    if (in < m->row_bytes) {
      const size_t e = std::min(end, r * m->stride + m->row_bytes);
      std::memcpy(dst + (pos - lo), src + r * m->row_bytes + in, e - pos);
      pos = e;
    }
    if (pos < end) {
      std::memset(dst + (pos - lo), 0, end - pos);
      pos = end;
    }
  }
}

// image_range over up to kCopyThreads host threads, each at least
// kCopySlice bytes.
constexpr size_t kCopyThreads = 8;

void image_range_parallel(const rh_matrix* m, const uint8_t* src, size_t lo, size_t hi, uint8_t* dst) {
  const size_t n = hi - lo;
  size_t threads = std::min<size_t>(kCopyThreads, std::max<size_t>(1, std::thread::hardware_concurrency()));
  threads = std::min(threads, std::max<size_t>(1, n / kCopySlice));
  if (threads <= 1) {
    image_range(m, src, lo, hi, dst);
    return;
  }
  const size_t part = round_up((n + threads - 1) / threads, 4096);
  std::vector<std::thread> pool;
  size_t done = std::min(hi, lo + part);  // the caller's own part
  for (size_t t = 1; t < threads && lo + t * part < hi; t++) {
    const size_t a = lo + t * part, b = std::min(hi, a + part);
    try {
      pool.emplace_back(image_range, m, src, a, b, dst + (a - lo));
    } catch (...) {  // no thread to spare: this one fills the rest
      done = a;
      break;
    }
    done = b;
  }
  image_range(m, src, lo, std::min(hi, lo + part), dst);
  if (done < hi) image_range(m, src, done, hi, dst + (done - lo));
  for (auto& th : pool) th.join();
}

struct Dma {
  uint8_t* dst;
  size_t off, len;
};

}  // namespace

// Every matrix's image goes through two pinned buffers: while the DMA engine
// copies one to HBM, host threads fill the other from the (pageable) source
// bytes. One synchronization at the end.
rh_status matrix_upload(rh_ctx* ctx, PendingUpload* p, size_t n) {
  if (!ctx || (!p && n)) return RH_ERR_INVALID_ARGUMENT;
  RH_HIP(ctx, hipSetDevice(ctx->device));
  if (!ctx->stage[0]) {
    for (int b = 0; b < 2; b++) {
      RH_HIP(ctx, hipHostMalloc(reinterpret_cast<void**>(&ctx->stage[b]), kStageBytes, hipHostMallocDefault));
      RH_HIP(ctx, hipEventCreateWithFlags(&ctx->stage_done[b], hipEventDisableTiming));
      RH_HIP(ctx, hipEventRecord(ctx->stage_done[b], ctx->stream));
    }
  }
  int cur = 0;
  size_t fill = 0;
  std::vector<Dma> dmas;
  auto flush = [&]() -> rh_status {
    for (const Dma& d : dmas)
      RH_HIP(ctx, hipMemcpyAsync(d.dst, ctx->stage[cur] + d.off, d.len, hipMemcpyHostToDevice, ctx->stream));
    RH_HIP(ctx, hipEventRecord(ctx->stage_done[cur], ctx->stream));
    dmas.clear();
    cur ^= 1;
    fill = 0;
    // the other buffer's copies must be done before it is refilled
    RH_HIP(ctx, hipEventSynchronize(ctx->stage_done[cur]));
    return RH_OK;
  };
  // the buffer about to be filled first may still feed a previous call's
  // copies only if that call failed midway; wait for it anyway
  RH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  for (size_t i = 0; i < n; i++) {
    rh_matrix* m = p[i].m;
    for (size_t off = 0; off < m->bytes;) {
      const size_t take = std::min(m->bytes - off, kStageBytes - fill);
      image_range_parallel(m, p[i].src, off, off + take, ctx->stage[cur] + fill);
      dmas.push_back({m->data + off, fill, take});
      fill += take;
      off += take;
      if (fill == kStageBytes) {
        rh_status st = flush();
        if (st != RH_OK) return st;
      }
    }
  }
  if (fill) {
    rh_status st = flush();
    if (st != RH_OK) return st;
  }
  RH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return RH_OK;
}
}  // namespace rh

extern "C" {

const char* rh_adapter_name(void) { return "hip-gfx950"; }

void rh_reload_tuning(void) { load_tuning(); }

rh_status rh_init(int device, rh_ctx** out) {
  if (!out) return RH_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) return RH_ERR_NO_DEVICE;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return RH_ERR_NO_DEVICE;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return RH_ERR_NO_DEVICE;
  rh_ctx* ctx = new (std::nothrow) rh_ctx();
  if (!ctx) return RH_ERR_OUT_OF_MEMORY;
  init_tuning();  // the first context reads the switches; rh_reload_tuning re-reads them
  ctx->device = device;
  if (hipSetDevice(device) != hipSuccess || hipStreamCreate(&ctx->stream) != hipSuccess) {
    delete ctx;
    return RH_ERR_DEVICE;
  }
  // the split GEMMs' arrival counters, zeroed once; without them split
  // GEMMs combine in a launch of their own
  if (hipMalloc(&ctx->tile_counters, kFixupTiles * sizeof(uint32_t)) != hipSuccess ||
      hipMemsetAsync(ctx->tile_counters, 0, kFixupTiles * sizeof(uint32_t), ctx->stream) != hipSuccess ||
      hipStreamSynchronize(ctx->stream) != hipSuccess) {
    (void)hipGetLastError();
    if (ctx->tile_counters) (void)hipFree(ctx->tile_counters);
    ctx->tile_counters = nullptr;
  }
  // the allocation-free entry point's array on this device; a failure only
  // disables that entry point (it reports the error)
  const hipError_t se = scratch_setup(device);
  if (se != hipSuccess) {
    (void)hipGetLastError();
    ctx->last_error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(se);
  }
  *out = ctx;
  return RH_OK;
}

void rh_destroy(rh_ctx* ctx) {
  if (!ctx) return;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  for (void* b : ctx->buf)
    if (b) hipFree(b);
  if (ctx->tile_counters) hipFree(ctx->tile_counters);
  for (int b = 0; b < 2; b++) {
    if (ctx->stage[b]) hipHostFree(ctx->stage[b]);
    if (ctx->stage_done[b]) hipEventDestroy(ctx->stage_done[b]);
  }
  hipStreamDestroy(ctx->stream);
  delete ctx;
}

const char* rh_last_error(const rh_ctx* ctx) { return ctx ? ctx->last_error.c_str() : rh::t_last_error.c_str(); }

void* rh_stream(rh_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

size_t rh_gemm_min_tokens(void) { return g_gemm_min_tokens; }
void rh_set_gemm_min_tokens(size_t tokens) { g_gemm_min_tokens = tokens; }

rh_status rh_matrix_load(rh_ctx* ctx, uint32_t type_id, const void* data, size_t len, size_t rows,
                         size_t cols, rh_matrix** out) {
  if (!ctx || !out || (!data && len)) return RH_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  PendingUpload p;
  rh_status st = matrix_prepare(ctx, type_id, data, len, rows, cols, &p);
  if (st != RH_OK) return st;
  st = matrix_upload(ctx, &p, 1);
  if (st != RH_OK) {
    rh_matrix_free(p.m);
    return st;
  }
  *out = p.m;
  return RH_OK;
}

// Frees without touching the context, which may already be destroyed: work
// queued on any stream may still read the matrix, so the device drains first.
void rh_matrix_free(rh_matrix* m) {
  if (!m) return;
  hipSetDevice(m->device);
  hipDeviceSynchronize();
  hipFree(m->data);
  delete m;
}

size_t rh_matrix_rows(const rh_matrix* m) { return m ? m->rows : 0; }
size_t rh_matrix_cols(const rh_matrix* m) { return m ? m->cols : 0; }
uint32_t rh_matrix_type(const rh_matrix* m) { return m ? m->type_id : 0; }
float rh_matrix_ternary_scale(const rh_matrix* m) { return m ? m->scale : 0.0f; }
size_t rh_matrix_device_bytes(const rh_matrix* m) {
  if (!m) return 0;
  return m->bytes;
}

rh_status rh_matrix_copy_row(rh_ctx* ctx, const rh_matrix* m, size_t index, float* out,
                             size_t out_len, int* found) {
  if (!ctx || !m || !found || (!out && out_len)) return RH_ERR_INVALID_ARGUMENT;
  *found = 0;
  if (index >= m->rows) return RH_OK;
  RH_HIP(ctx, hipSetDevice(ctx->device));
  const uint8_t* row = m->data + index * m->stride;
  if (m->type_id == RH_TYPE_F32) {
    // a dense row is copied whole into an output of its length (weights.rs:122-125)
    if (out_len < m->cols) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "output shorter than the row");
    RH_HIP(ctx, hipMemcpyAsync(out, row, m->cols * 4, hipMemcpyDeviceToHost, ctx->stream));
    RH_HIP(ctx, hipStreamSynchronize(ctx->stream));
    *found = 1;
    return RH_OK;
  }
  // Blocks: whole blocks the output holds (format.rs:219-226). Ternary: the
  // first min(cols, out_len) values, decoded as whole blocks and then all
  // multiplied by the tensor scale (weights.rs:134-147).
  const size_t bs = m->type_id == RH_TYPE_I2_S ? 128 : 256;
  const size_t span = m->type_id == RH_TYPE_I2_S ? (m->cols < out_len ? m->cols : out_len) : out_len;
  size_t nb = span / bs;
  if (nb > m->nblocks) nb = m->nblocks;
  rh_status st = ensure(ctx, kOut, (nb * bs + 1) * 4);
  if (st != RH_OK) return st;
  float* d = static_cast<float*>(ctx->buf[kOut]);
  if (nb) {
    RH_HIP(ctx, launch_dequantize_row(m->type_id, m->data, matrix_pitch(m), static_cast<uint32_t>(index),
                                      static_cast<uint32_t>(nb), m->scale, d, nb * bs, ctx->stream));
    RH_HIP(ctx, hipMemcpyAsync(out, d, nb * bs * 4, hipMemcpyDeviceToHost, ctx->stream));
  }
  RH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  if (m->type_id == RH_TYPE_I2_S)
    for (size_t i = nb * bs; i < span; i++) out[i] *= m->scale;
  *found = 1;
  return RH_OK;
}

rh_status rh_matmul_batch_device(rh_ctx* ctx, const float* inputs, size_t inputs_len, size_t tokens,
                                 const rh_job* jobs, size_t n_jobs, void* stream) {
  if (!ctx || (!jobs && n_jobs)) return RH_ERR_INVALID_ARGUMENT;
  if (tokens == 0 || tokens > inputs_len) return RH_OK;  // matmul.rs:230-232
  if (!inputs) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "no inputs");
  RH_HIP(ctx, hipSetDevice(ctx->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
  return run_batch(ctx, inputs, inputs_len, tokens, jobs, n_jobs, s, nullptr);
}

rh_status rh_matmul_batch_device_noalloc(rh_ctx* ctx, const float* inputs, size_t inputs_len, size_t tokens,
                                         const rh_job* jobs, size_t n_jobs, void* stream) {
  if (!ctx || (!jobs && n_jobs)) return RH_ERR_INVALID_ARGUMENT;
  if (tokens == 0 || tokens > inputs_len) return RH_OK;  // matmul.rs:230-232
  if (!inputs) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "no inputs");
  const size_t width = inputs_len / tokens;
  const size_t need = q8_layout_bytes(width, tokens);
  if (need > kScratchBytes)
    return fail(ctx, RH_ERR_INVALID_ARGUMENT,
                "the batch's quantized activations need " + std::to_string(need) +
                    " bytes; rh_matmul_batch_device_noalloc holds " + std::to_string(kScratchBytes));
  uint8_t* base = static_cast<uint8_t*>(scratch_ptr(ctx->device));
  if (!base) return fail(ctx, RH_ERR_DEVICE, "the allocation-free scratch has no address on this device");
  RH_HIP(ctx, hipSetDevice(ctx->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
  Q8Dev q[2];
  q8_layout(base, width, tokens, q);
  return run_batch(ctx, inputs, inputs_len, tokens, jobs, n_jobs, s, nullptr, q);
}

rh_status rh_matmul_batch_device_repeat(rh_ctx* ctx, const float* inputs, size_t inputs_len, size_t tokens,
                                        const rh_matrix* const* matrices, size_t n_matrices, float* out,
                                        size_t out_len, size_t launches, void* stream) {
  if (!ctx || (!matrices && launches) || (n_matrices == 0 && launches)) return RH_ERR_INVALID_ARGUMENT;
  for (size_t i = 0; i < launches; i++) {
    const rh_job job{matrices[i % n_matrices], out, out_len};
    const rh_status st = rh_matmul_batch_device(ctx, inputs, inputs_len, tokens, &job, 1, stream);
    if (st != RH_OK) return st;
  }
  return RH_OK;
}

rh_status rh_matmul_batch(rh_ctx* ctx, const float* inputs, size_t inputs_len, size_t tokens,
                          const rh_job* jobs, size_t n_jobs) {
  if (!ctx || (!jobs && n_jobs)) return RH_ERR_INVALID_ARGUMENT;
  if (tokens == 0 || tokens > inputs_len) return RH_OK;
  if (!inputs) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "no inputs");
  RH_HIP(ctx, hipSetDevice(ctx->device));
  size_t total_out = 0;
  std::vector<size_t> written(n_jobs);
  for (size_t i = 0; i < n_jobs; i++) {
    if (!jobs[i].weights) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "a job has no matrix");
    const size_t rows = rows_for(jobs[i].weights, jobs[i].out_len, tokens);
    const size_t w = rows * tokens < jobs[i].out_len ? rows * tokens : jobs[i].out_len;
    written[i] = w;
    total_out += round_up(w + 1, 64);
  }
  rh_status st;
  if ((st = ensure(ctx, kIn, inputs_len * sizeof(float))) != RH_OK) return st;
  if ((st = ensure(ctx, kOut, total_out * sizeof(float))) != RH_OK) return st;
  float* d_in = static_cast<float*>(ctx->buf[kIn]);
  float* d_out = static_cast<float*>(ctx->buf[kOut]);
  RH_HIP(ctx, hipMemcpyAsync(d_in, inputs, inputs_len * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  std::vector<rh_job> dj(jobs, jobs + n_jobs);
  size_t off = 0;
  for (size_t i = 0; i < n_jobs; i++) {
    dj[i].out = d_out + off;
    off += round_up(written[i] + 1, 64);
  }
  if ((st = run_batch(ctx, d_in, inputs_len, tokens, dj.data(), n_jobs, ctx->stream, nullptr)) != RH_OK)
    return st;
  for (size_t i = 0; i < n_jobs; i++)
    if (written[i])
      RH_HIP(ctx, hipMemcpyAsync(jobs[i].out, dj[i].out, written[i] * sizeof(float), hipMemcpyDeviceToHost,
                                 ctx->stream));
  RH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return RH_OK;
}

rh_status rh_matvec_batch(rh_ctx* ctx, const float* input, size_t len, const rh_job* jobs, size_t n_jobs) {
  return rh_matmul_batch(ctx, input, len, 1, jobs, n_jobs);
}

rh_status rh_q8_new(rh_ctx* ctx, rh_q8** out) {
  if (!ctx || !out) return RH_ERR_INVALID_ARGUMENT;
  *out = new (std::nothrow) rh_q8();
  if (!*out) return fail(ctx, RH_ERR_OUT_OF_MEMORY, "host allocation failed");
  (*out)->ctx = ctx;
  (*out)->device = ctx->device;
  return RH_OK;
}

void rh_q8_free(rh_q8* q) {
  if (!q) return;
  if (q->mem) {
    hipSetDevice(q->device);
    hipDeviceSynchronize();
    hipFree(q->mem);
  }
  delete q;
}

rh_status rh_q8_quantize_device(rh_ctx* ctx, rh_q8* q, int kind, const float* inputs, size_t inputs_len,
                                size_t tokens, void* stream) {
  if (!ctx || !q) return RH_ERR_INVALID_ARGUMENT;
  if (kind != RH_Q8_SUPER_BLOCK && kind != RH_Q8_ROW)
    return fail(ctx, RH_ERR_INVALID_ARGUMENT, "unknown activation kind");
  if (tokens == 0 || tokens > inputs_len) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "no whole token");
  if (!inputs) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "no inputs");
  RH_HIP(ctx, hipSetDevice(ctx->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
  const size_t width = inputs_len / tokens;
  const size_t qstride = round_up(width < 256 ? 256 : width, 256);
  const size_t bstride = round_up(qstride / 32, 8);
  const size_t need = tokens * qstride + 4 * tokens * bstride * (1 + 1 + 2) + 1024;
  if (q->cap < need) {
    if (q->mem) {
      RH_HIP(ctx, hipDeviceSynchronize());
      RH_HIP(ctx, hipFree(q->mem));
      q->mem = nullptr;
      q->cap = 0;
    }
    RH_HIP(ctx, hipMalloc(&q->mem, need));
    q->cap = need;
  }
  uint8_t* base = static_cast<uint8_t*>(q->mem);
  q->q.qstride = qstride;
  q->q.bstride = bstride;
  q->q.quants = reinterpret_cast<int8_t*>(base);
  q->q.scales = reinterpret_cast<float*>(base + tokens * qstride);
  q->q.sums = reinterpret_cast<int32_t*>(base + tokens * qstride + 4 * tokens * bstride);
  q->q.sums16 = reinterpret_cast<int32_t*>(base + tokens * qstride + 8 * tokens * bstride);
  q->q.n_blocks = kind == RH_Q8_SUPER_BLOCK ? width / 256 * 8 : width / 32;
  q->kind = kind;
  q->width = width;
  q->tokens = tokens;
  if (kind == RH_Q8_SUPER_BLOCK) RH_HIP(ctx, launch_quantize_super(inputs, width, tokens, q->q, s));
  else RH_HIP(ctx, launch_quantize_row(inputs, width, tokens, q->q, s));
  return RH_OK;
}

rh_status rh_dot_matrix_device(rh_ctx* ctx, const rh_matrix* m, const rh_q8* q, float* out, size_t out_len,
                               void* stream) {
  if (!ctx || !m || !q || (!out && out_len)) return RH_ERR_INVALID_ARGUMENT;
  if (q->tokens == 0) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "the activation holds no token");
  const int want = m->type_id == RH_TYPE_I2_S ? RH_Q8_ROW : RH_Q8_SUPER_BLOCK;
  if (!is_kquant(m->type_id) && m->type_id != RH_TYPE_I2_S)
    return fail(ctx, RH_ERR_INVALID_ARGUMENT, "dense rows take f32 inputs: use rh_matmul_batch_device");
  if (q->kind != want) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "activation kind does not match the format");
  RH_HIP(ctx, hipSetDevice(ctx->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
  rh_job job{m, out, out_len};
  return launch_jobs(ctx, nullptr, q->width, q->tokens, &job, 1, q->q, q->q, s, nullptr, 0u);
}

rh_status rh_quantize(rh_ctx* ctx, int kind, const float* x, size_t len, int8_t* quants, float* scales,
                      int32_t* sums, size_t* n_blocks) {
  if (!ctx || !n_blocks || (!x && len)) return RH_ERR_INVALID_ARGUMENT;
  if (kind != RH_Q8_SUPER_BLOCK && kind != RH_Q8_ROW)
    return fail(ctx, RH_ERR_INVALID_ARGUMENT, "unknown activation kind");
  RH_HIP(ctx, hipSetDevice(ctx->device));
  const size_t nb = kind == RH_Q8_SUPER_BLOCK ? len / 256 * 8 : len / 32;
  *n_blocks = nb;
  if (nb == 0) return RH_OK;
  if (!quants || !scales || !sums) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "null output");
  rh_status st;
  if ((st = ensure(ctx, kIn, len * sizeof(float))) != RH_OK) return st;
  if ((st = ensure_q8(ctx, len, 1)) != RH_OK) return st;
  float* d_in = static_cast<float*>(ctx->buf[kIn]);
  RH_HIP(ctx, hipMemcpyAsync(d_in, x, len * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  const Q8Dev& q = kind == RH_Q8_SUPER_BLOCK ? ctx->super_q : ctx->row_q;
  if (kind == RH_Q8_SUPER_BLOCK) RH_HIP(ctx, launch_quantize_super(d_in, len, 1, q, ctx->stream));
  else RH_HIP(ctx, launch_quantize_row(d_in, len, 1, q, ctx->stream));
  RH_HIP(ctx, hipMemcpyAsync(quants, q.quants, nb * 32, hipMemcpyDeviceToHost, ctx->stream));
  RH_HIP(ctx, hipMemcpyAsync(scales, q.scales, nb * 4, hipMemcpyDeviceToHost, ctx->stream));
  RH_HIP(ctx, hipMemcpyAsync(sums, q.sums, nb * 4, hipMemcpyDeviceToHost, ctx->stream));
  RH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return RH_OK;
}

rh_status rh_ternary_dot_i32(rh_ctx* ctx, const rh_matrix* m, const float* inputs, size_t inputs_len,
                             size_t tokens, int32_t* out, size_t out_len) {
  if (!ctx || !m || (!out && out_len)) return RH_ERR_INVALID_ARGUMENT;
  if (m->type_id != RH_TYPE_I2_S) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "not an I2_S matrix");
  if (tokens == 0 || tokens > inputs_len) return RH_OK;
  if (!inputs) return fail(ctx, RH_ERR_INVALID_ARGUMENT, "no inputs");
  RH_HIP(ctx, hipSetDevice(ctx->device));
  const size_t rows = rows_for(m, out_len, tokens);
  const size_t w = rows * tokens < out_len ? rows * tokens : out_len;
  rh_status st;
  if ((st = ensure(ctx, kIn, inputs_len * sizeof(float))) != RH_OK) return st;
  if ((st = ensure(ctx, kRaw, (w + 1) * sizeof(int32_t))) != RH_OK) return st;
  float* d_in = static_cast<float*>(ctx->buf[kIn]);
  int32_t* d_raw = static_cast<int32_t*>(ctx->buf[kRaw]);
  RH_HIP(ctx, hipMemcpyAsync(d_in, inputs, inputs_len * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  rh_job job{m, reinterpret_cast<float*>(d_raw), out_len};
  if ((st = run_batch(ctx, d_in, inputs_len, tokens, &job, 1, ctx->stream, d_raw)) != RH_OK) return st;
  if (w) RH_HIP(ctx, hipMemcpyAsync(out, d_raw, w * sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
  RH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return RH_OK;
}

}  // extern "C"
