// C ABI of libccq_hip.so: argument checks, buffer carving, kernel launches.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/ccq_hip.h"
#include "ccq_params.h"

namespace ccq {
hipError_t launch_clean_fwd(const CleanFwdArgs& a, int K, hipStream_t st);
hipError_t launch_clean_bwd(const CleanBwdArgs& a, int K, hipStream_t st);
hipError_t launch_lam_reduce(const LamReduceArgs& a, hipStream_t st);
hipError_t launch_sum_rows(const float* part, float* out, int nblk, int cols, hipStream_t st);
hipError_t launch_gdn_stage(int stage, const GdnArgs& a, int K, int V, hipStream_t st);
hipError_t launch_l2norm_fwd(const L2NormArgs& a, hipStream_t st);
hipError_t launch_l2norm_bwd(const L2NormArgs& a, hipStream_t st);
hipError_t launch_chunk_index(const int64_t* cu, int N, int* chunk_off, int* chunk_idx, int cap, hipStream_t st);
}  // namespace ccq

using namespace ccq;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return CCQ_OK;
  return fail(CCQ_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Consecutive sub-buffers of a caller-provided byte buffer.
struct Slicer {
  char* base;
  size_t off = 0;
  template <typename T>
  T* take(size_t n) {
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += align256(n * sizeof(T));
    return p;
  }
};

int check_common(int B, int T, int H, int N, const int64_t* cu) {
  if (B < 0 || T < 0 || H <= 0 || N < 0) return fail(CCQ_ERR_SHAPE, "negative or zero size (B=%d T=%d H=%d N=%d)", B, T, H, N);
  if (cu && B != 1) return fail(CCQ_ERR_SHAPE, "varlen inputs need B == 1 (got B=%d)", B);
  if (!cu && N != B) return fail(CCQ_ERR_SHAPE, "dense inputs need N == B (got N=%d, B=%d)", N, B);
  return CCQ_OK;
}

int clean_k_ok(int K) { return K == 32 || K == 64 || K == 128 || K == 256; }

// ---- optional kernel timing (measurement only; off unless ccq_timing_enable(1)) ----
struct TimingState {
  std::mutex mu;
  bool on = false;
  std::map<std::string, std::vector<std::pair<hipEvent_t, hipEvent_t>>> pending;
  std::map<std::string, std::pair<double, int64_t>> done;
};

TimingState& timing() {
  static TimingState t;
  return t;
}

// Run `launch` between two events recorded on `st` when timing is enabled.
template <typename F>
hipError_t timed(const char* name, hipStream_t st, F&& launch) {
  TimingState& t = timing();
  {
    std::lock_guard<std::mutex> g(t.mu);
    if (!t.on) return launch();
  }
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess) return launch();
  if (hipEventCreate(&b) != hipSuccess) {
    (void)hipEventDestroy(a);
    return launch();
  }
  (void)hipEventRecord(a, st);
  const hipError_t e = launch();
  (void)hipEventRecord(b, st);
  std::lock_guard<std::mutex> g(t.mu);
  t.pending[name].push_back({a, b});
  return e;
}

void resolve_pending(TimingState& t) {
  for (auto& kv : t.pending) {
    auto& acc = t.done[kv.first];
    for (auto& ev : kv.second) {
      float ms = 0.f;
      if (hipEventSynchronize(ev.second) == hipSuccess && hipEventElapsedTime(&ms, ev.first, ev.second) == hipSuccess) {
        acc.first += ms;
        acc.second += 1;
      }
      (void)hipEventDestroy(ev.first);
      (void)hipEventDestroy(ev.second);
    }
  }
  t.pending.clear();
}

}  // namespace

extern "C" {

int ccq_abi_version(void) { return 1; }

const char* ccq_last_error(void) { return g_err; }

int ccq_clean_fwd(const void* q, const void* k, const float* lambda, const float* gate_w, const float* gate_b,
                  float* lambda_out, const float* h0, const float* m0, const int64_t* cu_seqlens, void* q_clean,
                  float* q_clean_f32, float* h_final, float* m_final, int B, int T, int H, int K, int N,
                  int position_offset, int subtract_mean, void* stream) {
  if (int s = check_common(B, T, H, N, cu_seqlens)) return s;
  if (!clean_k_ok(K)) return fail(CCQ_ERR_SHAPE, "ccq_clean_fwd: K=%d not in {32, 64, 128, 256}", K);
  if (!q || !k) return fail(CCQ_ERR_NULL, "ccq_clean_fwd: q and k are required");
  if (!gate_w && !lambda) return fail(CCQ_ERR_NULL, "ccq_clean_fwd: lambda or gate_w is required");
  if (gate_w && !gate_b) return fail(CCQ_ERR_NULL, "ccq_clean_fwd: gate_w needs gate_b");
  if (!q_clean && !q_clean_f32) return fail(CCQ_ERR_NULL, "ccq_clean_fwd: no output (q_clean / q_clean_f32)");
  if (!aligned16(q) || !aligned16(k)) return fail(CCQ_ERR_ALIGN, "ccq_clean_fwd: q/k must be 16-byte aligned");
  CleanFwdArgs a{};
  a.q = q; a.k = k; a.lam = lambda; a.gate_w = gate_w; a.gate_b = gate_b; a.lam_out = lambda_out;
  a.h0 = h0; a.m0 = m0; a.cu = cu_seqlens; a.qc = q_clean; a.qc32 = q_clean_f32; a.h_fin = h_final;
  a.m_fin = m_final; a.T = T; a.H = H; a.N = N; a.pos_off = position_offset; a.subtract_mean = subtract_mean ? 1 : 0;
  hipStream_t st = (hipStream_t)stream;
  return hip_status(timed("clean_fwd", st, [&] { return launch_clean_fwd(a, K, st); }), "ccq_clean_fwd");
}

size_t ccq_clean_bwd_workspace_bytes(int64_t tokens, int H, int K, int gate) {
  const size_t ncb = (size_t)(K / 32);
  size_t s = align256(ncb * (size_t)tokens * H * sizeof(float));
  if (gate) {
    const size_t nblk = (size_t)((tokens + 63) / 64);
    s += align256((size_t)tokens * H * K * sizeof(float));    // dq of the cleaning path (fp32)
    s += align256(nblk * H * K * sizeof(float));               // dW partials
    s += align256(nblk * H * sizeof(float));                   // db partials
    s += align256((size_t)tokens * H * sizeof(float));         // dlambda
  }
  return s;
}

int ccq_clean_bwd(const void* q, const void* k, const float* lambda, const float* gate_w, const float* gate_b,
                  const float* dq_clean_f32, const void* dq_clean, const float* dk_extra, const float* h0,
                  const float* m0, const float* m_end, const int64_t* cu_seqlens, const float* dh_final,
                  const float* dm_final, void* dq, float* dq_f32, void* dk, float* dk_f32, float* dlambda,
                  float* dgate_w, float* dgate_b, float* dh0, float* dm0, void* workspace, int B, int T, int H,
                  int K, int N, int position_offset, int subtract_mean, void* stream) {
  if (int s = check_common(B, T, H, N, cu_seqlens)) return s;
  if (!clean_k_ok(K)) return fail(CCQ_ERR_SHAPE, "ccq_clean_bwd: K=%d not in {32, 64, 128, 256}", K);
  if (!q || !k || !lambda || !workspace) return fail(CCQ_ERR_NULL, "ccq_clean_bwd: q, k, lambda, workspace are required");
  if (!dq_clean_f32 && !dq_clean) return fail(CCQ_ERR_NULL, "ccq_clean_bwd: upstream gradient missing");
  if (subtract_mean && !m_end) return fail(CCQ_ERR_NULL, "ccq_clean_bwd: m_end is required when subtract_mean");
  if (!dq && !dq_f32) return fail(CCQ_ERR_NULL, "ccq_clean_bwd: no dq output");
  if (!dk && !dk_f32) return fail(CCQ_ERR_NULL, "ccq_clean_bwd: no dk output");
  const bool gate = gate_w != nullptr;
  if (gate && (!gate_b || !dgate_w || !dgate_b)) return fail(CCQ_ERR_NULL, "ccq_clean_bwd: gate needs gate_b, dgate_w, dgate_b");
  const long tokens = (long)B * T;  // varlen: B == 1 and T is the packed length
  const int ncb = K / 32;
  Slicer sl{(char*)workspace};
  float* dlam_part = sl.take<float>((size_t)ncb * tokens * H);
  float* dq32_ws = nullptr;
  float* dw_part = nullptr;
  float* db_part = nullptr;
  float* dlam_ws = nullptr;
  const int nblk = (int)((tokens + 63) / 64);
  if (gate) {
    dq32_ws = sl.take<float>((size_t)tokens * H * K);
    dw_part = sl.take<float>((size_t)nblk * H * K);
    db_part = sl.take<float>((size_t)nblk * H);
    dlam_ws = sl.take<float>((size_t)tokens * H);
  }
  hipStream_t st = (hipStream_t)stream;
  CleanBwdArgs a{};
  a.q = q; a.k = k; a.lam = lambda; a.dqc32 = dq_clean_f32; a.dqc16 = dq_clean_f32 ? nullptr : dq_clean;
  a.dk_extra = dk_extra; a.h0 = h0; a.m0 = m0; a.m_end = m_end; a.cu = cu_seqlens; a.dh_fin = dh_final;
  a.dm_fin = dm_final; a.dk = dk; a.dk32 = dk_f32; a.dlam_part = dlam_part; a.dh0 = dh0; a.dm0 = dm0;
  a.ntok = tokens; a.T = T; a.H = H; a.N = N; a.pos_off = position_offset; a.subtract_mean = subtract_mean ? 1 : 0;
  if (gate) {
    a.dq = nullptr;
    a.dq32 = dq32_ws;
  } else {
    a.dq = dq;
    a.dq32 = dq_f32;
  }
  if (int s = hip_status(timed("clean_bwd", st, [&] { return launch_clean_bwd(a, K, st); }), "ccq_clean_bwd"))
    return s;
  LamReduceArgs r{};
  r.dlam_part = dlam_part; r.lam = lambda; r.q = q; r.gate_w = gate_w; r.dq32 = dq32_ws;
  r.dlam = gate ? (dlambda ? dlambda : dlam_ws) : dlambda;
  r.dq = gate ? dq : nullptr; r.dq_out32 = gate ? dq_f32 : nullptr;
  r.dw_part = dw_part; r.db_part = db_part; r.ntok = tokens; r.H = H; r.K = K; r.ncb = ncb;
  if (r.dlam || gate) {
    if (int s = hip_status(timed("lam_reduce", st, [&] { return launch_lam_reduce(r, st); }), "ccq_clean_bwd(dlambda)"))
      return s;
  }
  if (gate) {
    if (int s = hip_status(launch_sum_rows(dw_part, dgate_w, nblk, H * K, st), "ccq_clean_bwd(dW)")) return s;
    if (int s = hip_status(launch_sum_rows(db_part, dgate_b, nblk, H, st), "ccq_clean_bwd(db)")) return s;
  }
  return CCQ_OK;
}

int ccq_chunk_index(const int64_t* cu_seqlens, int N, int* chunk_offsets, int* chunk_index, int capacity,
                    void* stream) {
  if (!cu_seqlens || !chunk_offsets || !chunk_index) return fail(CCQ_ERR_NULL, "ccq_chunk_index: null pointer");
  if (N < 0 || capacity < 0) return fail(CCQ_ERR_SHAPE, "ccq_chunk_index: bad sizes");
  return hip_status(launch_chunk_index(cu_seqlens, N, chunk_offsets, chunk_index, capacity, (hipStream_t)stream),
                    "ccq_chunk_index");
}

}  // extern "C"

namespace {

struct GdnSaved {
  float* gcum;
  float* tmat;
  void* w;
  float* u;
  void* hT;
  void* hTl;
  float* U;
  float* PT;
};

size_t carve_saved(char* base, int64_t tokens, int NTG, int H, int K, int V, GdnSaved* s) {
  Slicer sl{base};
  GdnSaved t;
  t.gcum = sl.take<float>((size_t)tokens * H);
  t.tmat = sl.take<float>((size_t)NTG * H * 64 * 64);
  t.w = sl.take<uint16_t>((size_t)tokens * H * K);
  t.u = sl.take<float>((size_t)tokens * H * V);
  t.hT = sl.take<uint16_t>((size_t)NTG * H * V * K);
  t.hTl = sl.take<uint16_t>((size_t)NTG * H * V * K);
  t.U = sl.take<float>((size_t)tokens * H * V);
  t.PT = sl.take<float>((size_t)NTG * H * 64 * 64);
  if (s) *s = t;
  return sl.off;
}

struct GdnWork {
  float* dU;
  void* dhT;
  void* dhTl;
  float* dkp32;
  float* dw32;
  float* dgp;
};

size_t carve_work(char* base, int64_t tokens, int NTG, int H, int K, int V, GdnWork* s) {
  Slicer sl{base};
  GdnWork t;
  t.dU = sl.take<float>((size_t)tokens * H * V);
  t.dhT = sl.take<uint16_t>((size_t)NTG * H * V * K);
  t.dhTl = sl.take<uint16_t>((size_t)NTG * H * V * K);
  t.dkp32 = sl.take<float>((size_t)tokens * H * K);
  t.dw32 = sl.take<float>((size_t)tokens * H * K);
  t.dgp = sl.take<float>((size_t)(K / 64) * tokens * H);
  if (s) *s = t;
  return sl.off;
}

int gdn_check(const char* who, int B, int T, int H, int K, int V, int N, const int64_t* cu, const int* chunk_index,
              const int* chunk_offsets, int num_chunks) {
  if (int s = check_common(B, T, H, N, cu)) return s;
  if (!(K == 64 || K == 128 || K == 256)) return fail(CCQ_ERR_SHAPE, "%s: K=%d not in {64, 128, 256}", who, K);
  if (V <= 0 || V % 64 != 0 || V > 1024) return fail(CCQ_ERR_SHAPE, "%s: V=%d must be a positive multiple of 64 (<= 1024)", who, V);
  if (cu && (!chunk_index || !chunk_offsets)) return fail(CCQ_ERR_NULL, "%s: varlen needs chunk_index and chunk_offsets", who);
  if (!cu && num_chunks != B * ((T + 63) / 64))
    return fail(CCQ_ERR_SHAPE, "%s: num_chunks=%d, expected B*ceil(T/64)=%d", who, num_chunks, B * ((T + 63) / 64));
  if (cu && num_chunks < 0) return fail(CCQ_ERR_SHAPE, "%s: negative num_chunks", who);
  return CCQ_OK;
}

}  // namespace

extern "C" {

size_t ccq_gdn_saved_bytes(int64_t tokens, int num_chunks, int H, int K, int V) {
  return carve_saved(nullptr, tokens, num_chunks, H, K, V, nullptr);
}

size_t ccq_gdn_bwd_workspace_bytes(int64_t tokens, int num_chunks, int H, int K, int V) {
  return carve_work(nullptr, tokens, num_chunks, H, K, V, nullptr);
}

int ccq_gdn_fwd(const void* q, const float* q_f32, const void* k, const void* v, const float* g, const float* beta,
                const float* initial_state, const int64_t* cu_seqlens, const int* chunk_index,
                const int* chunk_offsets, int num_chunks, void* o, float* final_state, void* saved, int B, int T,
                int H, int K, int V, int N, float scale, void* stream) {
  if (int s = gdn_check("ccq_gdn_fwd", B, T, H, K, V, N, cu_seqlens, chunk_index, chunk_offsets, num_chunks)) return s;
  if ((!q && !q_f32) || !k || !v || !beta || !o || !saved) return fail(CCQ_ERR_NULL, "ccq_gdn_fwd: null input/output");
  if (!aligned16(q) || !aligned16(q_f32) || !aligned16(k) || !aligned16(v) || !aligned16(saved))
    return fail(CCQ_ERR_ALIGN, "ccq_gdn_fwd: tensors must be 16-byte aligned");
  const int64_t tokens = (int64_t)B * T;
  GdnSaved sv;
  carve_saved((char*)saved, tokens, num_chunks, H, K, V, &sv);
  GdnArgs a{};
  a.qc16 = q_f32 ? nullptr : q; a.qc32 = q_f32; a.k = k; a.v = v; a.g = g; a.beta = beta; a.s0 = initial_state;
  a.cu = cu_seqlens; a.chunk_idx = chunk_index; a.chunk_off = chunk_offsets;
  a.gcum = sv.gcum; a.tmat = sv.tmat; a.w = sv.w; a.u = sv.u; a.hT = sv.hT; a.hTl = sv.hTl; a.U = sv.U; a.PT = sv.PT;
  a.o = o; a.s_fin = final_state; a.scale = scale;
  a.T = T; a.H = H; a.N = N; a.NT = (T + 63) / 64; a.NTG = num_chunks;
  hipStream_t st = (hipStream_t)stream;
  static const char* names[] = {"gdn_prep", "gdn_fwd_state", "gdn_fwd_o"};
  const int stages[] = {kGdnPrep, kGdnFwdState, kGdnFwdO};
  for (int i = 0; i < 3; ++i) {
    if (int s = hip_status(timed(names[i], st, [&] { return launch_gdn_stage(stages[i], a, K, V, st); }), names[i]))
      return s;
  }
  return CCQ_OK;
}

int ccq_gdn_bwd(const void* q, const float* q_f32, const void* k, const void* v, const float* g, const float* beta,
                const int64_t* cu_seqlens, const int* chunk_index, const int* chunk_offsets, int num_chunks,
                const void* saved, const void* d_o, const float* d_final_state, void* workspace, float* dq_f32,
                float* dk_f32, void* dv, float* dbeta, float* dg, float* d_initial_state, int B, int T, int H, int K,
                int V, int N, float scale, void* stream) {
  if (int s = gdn_check("ccq_gdn_bwd", B, T, H, K, V, N, cu_seqlens, chunk_index, chunk_offsets, num_chunks)) return s;
  if ((!q && !q_f32) || !k || !v || !beta || !saved || !d_o || !workspace || !dq_f32 || !dk_f32 || !dv || !dbeta ||
      !dg)
    return fail(CCQ_ERR_NULL, "ccq_gdn_bwd: null input/output");
  const int64_t tokens = (int64_t)B * T;
  GdnSaved sv;
  carve_saved((char*)saved, tokens, num_chunks, H, K, V, &sv);
  GdnWork wk;
  carve_work((char*)workspace, tokens, num_chunks, H, K, V, &wk);
  GdnArgs a{};
  a.qc16 = q_f32 ? nullptr : q; a.qc32 = q_f32; a.k = k; a.v = v; a.g = g; a.beta = beta;
  a.cu = cu_seqlens; a.chunk_idx = chunk_index; a.chunk_off = chunk_offsets;
  a.gcum = sv.gcum; a.tmat = sv.tmat; a.w = sv.w; a.u = sv.u; a.hT = sv.hT; a.hTl = sv.hTl; a.U = sv.U; a.PT = sv.PT;
  a.dout = d_o; a.ds_fin = d_final_state; a.dU = wk.dU; a.dhT = wk.dhT; a.dhTl = wk.dhTl; a.dq32 = dq_f32; a.dkp32 = wk.dkp32;
  a.dw32 = wk.dw32; a.dgp = wk.dgp; a.dk32 = dk_f32; a.dv = dv; a.dbeta = dbeta; a.dg = dg; a.ds0 = d_initial_state;
  a.scale = scale; a.T = T; a.H = H; a.N = N; a.NT = (T + 63) / 64; a.NTG = num_chunks;
  hipStream_t st = (hipStream_t)stream;
  static const char* names[] = {"gdn_bwd_state", "gdn_bwd_dqkw", "gdn_bwd_wy"};
  const int stages[] = {kGdnBwdState, kGdnBwdDqkw, kGdnBwdWy};
  for (int i = 0; i < 3; ++i) {
    if (int s = hip_status(timed(names[i], st, [&] { return launch_gdn_stage(stages[i], a, K, V, st); }), names[i]))
      return s;
  }
  return CCQ_OK;
}

int ccq_l2norm_fwd(const void* x, void* y, float* rstd, int64_t rows, int D, float eps, void* stream) {
  if (!x || !y) return fail(CCQ_ERR_NULL, "ccq_l2norm_fwd: null pointer");
  if (D <= 0 || D > 512 || rows < 0) return fail(CCQ_ERR_SHAPE, "ccq_l2norm_fwd: bad sizes rows=%lld D=%d", (long long)rows, D);
  L2NormArgs a{};
  a.x = x; a.y = y; a.rstd = rstd; a.rows = rows; a.D = D; a.eps = eps;
  return hip_status(launch_l2norm_fwd(a, (hipStream_t)stream), "ccq_l2norm_fwd");
}

int ccq_l2norm_bwd(const void* x, const float* rstd, const float* dy_f32, const void* dy, void* dx, int64_t rows,
                   int D, void* stream) {
  if (!x || !rstd || !dx || (!dy_f32 && !dy)) return fail(CCQ_ERR_NULL, "ccq_l2norm_bwd: null pointer");
  if (D <= 0 || D > 512 || rows < 0) return fail(CCQ_ERR_SHAPE, "ccq_l2norm_bwd: bad sizes");
  L2NormArgs a{};
  a.x = x; a.rstd = const_cast<float*>(rstd); a.dy32 = dy_f32; a.dy16 = dy_f32 ? nullptr : dy; a.dx = dx; a.rows = rows; a.D = D;
  return hip_status(launch_l2norm_bwd(a, (hipStream_t)stream), "ccq_l2norm_bwd");
}

}  // extern "C"

extern "C" {

int ccq_timing_enable(int on) {
  TimingState& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  t.on = on != 0;
  return CCQ_OK;
}

int ccq_timing_reset(void) {
  TimingState& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  resolve_pending(t);
  t.done.clear();
  return CCQ_OK;
}

int ccq_timing_read(const char* kernel, double* total_ms, int64_t* launches) {
  if (!kernel || !total_ms || !launches) return fail(CCQ_ERR_NULL, "ccq_timing_read: null pointer");
  TimingState& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  resolve_pending(t);
  auto it = t.done.find(kernel);
  *total_ms = it == t.done.end() ? 0.0 : it->second.first;
  *launches = it == t.done.end() ? 0 : it->second.second;
  return CCQ_OK;
}

}  // extern "C"
