// extern "C" entry points of libgdn2_hip.so (declared in include/gdn2_hip.h).
// Arguments are validated here, before anything is launched.
#include "../../include/gdn2_hip.h"
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"
#include "gdn2_layer.h"

namespace gdn2 {
hipError_t launch_decode(const void*, const void*, const void*, const float*, const void*,
                         const void*, float*, void*, int, int, int, int, int, long, long, int,
                         float, int, int, hipStream_t);
hipError_t launch_chunk_local(const void*, const void*, const void*, const float*, int, int, int,
                              int, long, long, int, long, float, unsigned short*, Varlen, hipStream_t);
hipError_t launch_scan(const void*, const void*, int, const unsigned short*, const float*, float*,
                       void*, int, int, int, int, int, int, long, long, int, long, Varlen, hipStream_t);
hipError_t launch_gemv(const void*, const void*, void*, int, int, int, int, long, long, hipStream_t);
size_t backward_workspace_bytes(int, int, int, int, int, long);
hipError_t launch_backward(const void*, const void*, const void*, const float*, const void*, const void*, int, float,
                           const float*, const void*, int, const float*, void*, void*, void*, float*, void*, void*,
                           float*, void*, int, int, int, int, int, long, hipStream_t);
size_t backward_varlen_workspace_bytes(int, int, int, int, int, long);
hipError_t launch_backward_varlen(const void*, const void*, const void*, const float*, const void*, const void*, int,
                                  float, const float*, const void*, int, const float*, void*, void*, void*, float*,
                                  void*, void*, float*, void*, const int*, int, int, int, int, int, long,
                                  hipStream_t);
}  // namespace gdn2

namespace {

constexpr int kAbiVersion = 4;   // 2: grouped key heads (HK); 3: packed sequences; 4: factored
                                 // DK = 128 records (58 112 B), packed training backward

bool dtype_ok(int dt) { return dt == GDN2_DTYPE_F32 || dt == GDN2_DTYPE_BF16 || dt == GDN2_DTYPE_F16; }

long record_elems(int DK) {
  if (DK == 64) return gdn2::ChunkLayout<64>::STRIDE;
  if (DK == 128) return gdn2::ChunkLayoutE<128>::STRIDE;
  return 0;
}

int status(hipError_t e) { return e == hipSuccess ? 0 : static_cast<int>(e); }

// shared checks of the prefill stages
int check_prefill(int B, int H, int DK, long s_alloc, long t0, long n_tokens) {
  if (B < 1 || H < 1 || t0 < 0 || n_tokens < 0 || s_alloc < t0 + n_tokens) return GDN2_ERR_ARG;
  if (DK != 64 && DK != 128) return GDN2_ERR_SHAPE;
  // a ragged last chunk is allowed: its rows past n_tokens are read as zeros
  if (static_cast<long>(B) * H * ((n_tokens + gdn2::kBS - 1) / gdn2::kBS) > 0x7fffffffL) return GDN2_ERR_SHAPE;
  return 0;
}

// record slots per key head of a packed batch: sequence s's chunk c sits at
// slot s + floor(cu[s] / 64) + c, which stays below ceil(T / 64) + nseq
long varlen_slots(int nseq, long T) { return (T + gdn2::kBS - 1) / gdn2::kBS + nseq; }

}  // namespace

extern "C" {

int gdn2_hip_version(void) { return kAbiVersion; }

const char* gdn2_hip_status_string(int s) {
  if (s == 0) return "success";
  if (s == GDN2_ERR_ARG) return "invalid argument (null pointer, negative size or bad dtype code)";
  if (s == GDN2_ERR_SHAPE) return "unsupported shape for the gfx950 kernels";
  if (s == GDN2_ERR_SCRATCH) return "the call needs more chunk records than the no-alloc scratch holds";
  if (s > 0) return hipGetErrorString(static_cast<hipError_t>(s));
  return "unknown status";
}

int gdn2_hip_decode(const void* q, const void* k, const void* v, const float* g, const void* b,
                    const void* w, int in_dtype, float* state, void* o, int out_dtype, int B,
                    int H, int HK, int DK, int DV, long s_alloc, long t0, long n, float scale,
                    void* stream) {
  if (!q || !k || !v || !g || !b || !w || !state || !o) return GDN2_ERR_ARG;
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return GDN2_ERR_ARG;
  if (B < 1 || H < 1 || HK < 1 || H % HK || n < 0 || t0 < 0 || s_alloc < t0 + n) return GDN2_ERR_ARG;
  if (DK != 32 && DK != 64 && DK != 128 && DK != 256) return GDN2_ERR_SHAPE;
  if (DV % 32 != 0 || DV > 4096) return GDN2_ERR_SHAPE;
  if (static_cast<long>(B) * H * (DV / 32) > 0x7fffffffL || n > 0x7fffffffL) return GDN2_ERR_SHAPE;
  return status(gdn2::launch_decode(q, k, v, g, b, w, state, o, B, H, HK, DK, DV, s_alloc, t0,
                                    static_cast<int>(n), scale, in_dtype, out_dtype,
                                    static_cast<hipStream_t>(stream)));
}

size_t gdn2_hip_prefill_workspace_bytes(int B, int HK, int DK, long n_tokens) {
  const long rec = record_elems(DK);
  if (rec == 0 || B < 1 || HK < 1 || n_tokens < 0) return 0;
  const long nc = (n_tokens + gdn2::kBS - 1) / gdn2::kBS;
  return static_cast<size_t>(B) * HK * nc * rec * 2;
}

int gdn2_hip_chunk_local(const void* q, const void* k, const void* b, const float* g,
                         int in_dtype, void* workspace, int B, int HK, int DK, long s_alloc,
                         long t0, long n_tokens, float scale, void* stream) {
  if (!q || !k || !b || !g || !workspace || !dtype_ok(in_dtype)) return GDN2_ERR_ARG;
  if (int e = check_prefill(B, HK, DK, s_alloc, t0, n_tokens)) return e;
  if (n_tokens == 0) return 0;
  return status(gdn2::launch_chunk_local(q, k, b, g, in_dtype, B, HK, DK, s_alloc, t0,
                                         static_cast<int>((n_tokens + gdn2::kBS - 1) / gdn2::kBS),
                                         n_tokens, scale,
                                         static_cast<unsigned short*>(workspace), gdn2::Varlen{nullptr, 0},
                                         static_cast<hipStream_t>(stream)));
}

int gdn2_hip_prefill_scan(const void* v, const void* w, int in_dtype, const void* workspace,
                          const float* state_in, float* state_out, void* o, int out_dtype, int B,
                          int H, int HK, int DK, int DV, long s_alloc, long t0, long n_tokens,
                          void* stream) {
  if (!v || !w || !workspace || !state_out || !o) return GDN2_ERR_ARG;
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return GDN2_ERR_ARG;
  if (HK < 1 || H % HK) return GDN2_ERR_ARG;
  if (int e = check_prefill(B, H, DK, s_alloc, t0, n_tokens)) return e;
  if (DV < 16 || DV % 16 || DV > 4096) return GDN2_ERR_SHAPE;
  if (n_tokens == 0) return GDN2_ERR_SHAPE;
  // the DK = 128 scan addresses a call's tokens with 32-bit byte offsets
  if (n_tokens * H * DV * 4 >= (1L << 31)) return GDN2_ERR_SHAPE;
  return status(gdn2::launch_scan(v, w, in_dtype, static_cast<const unsigned short*>(workspace),
                                  state_in, state_out, o, out_dtype, B, H, HK, DK, DV, s_alloc, t0,
                                  static_cast<int>((n_tokens + gdn2::kBS - 1) / gdn2::kBS), n_tokens,
                                  gdn2::Varlen{nullptr, 0}, static_cast<hipStream_t>(stream)));
}

int gdn2_hip_prefill_chunks(const void* q, const void* k, const void* v, const float* g,
                            const void* b, const void* w, int in_dtype, const float* state_in,
                            float* state_out, void* o, int out_dtype, void* workspace, int B,
                            int H, int HK, int DK, int DV, long s_alloc, long t0, long n_tokens,
                            float scale, void* stream) {
  if (!q || !k || !b || !g) return GDN2_ERR_ARG;
  if (!v || !w || !workspace || !state_out || !o) return GDN2_ERR_ARG;
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return GDN2_ERR_ARG;
  if (int e = check_prefill(B, H, DK, s_alloc, t0, n_tokens)) return e;
  if (DV < 16 || DV % 16 || DV > 4096 || n_tokens == 0) return GDN2_ERR_SHAPE;
  if (HK < 1 || H % HK) return GDN2_ERR_ARG;
  int s = gdn2_hip_chunk_local(q, k, b, g, in_dtype, workspace, B, HK, DK, s_alloc, t0, n_tokens,
                               scale, stream);
  if (s) return s;
  return gdn2_hip_prefill_scan(v, w, in_dtype, workspace, state_in, state_out, o, out_dtype, B, H,
                               HK, DK, DV, s_alloc, t0, n_tokens, stream);
}

size_t gdn2_hip_prefill_varlen_workspace_bytes(int nseq, int HK, int DK, long T) {
  const long rec = record_elems(DK);
  if (nseq < 1 || T < 0 || rec == 0 || HK < 1) return 0;
  return static_cast<size_t>(HK) * varlen_slots(nseq, T) * rec * 2;   // chunk records
}

int gdn2_hip_prefill_varlen(const void* q, const void* k, const void* v, const float* g,
                            const void* b, const void* w, int in_dtype, const int* cu_seqlens, int nseq,
                            const float* state_in, float* state_out, void* o, int out_dtype,
                            void* workspace, int H, int HK, int DK, int DV, long T, float scale,
                            void* stream) {
  if (!q || !k || !v || !g || !b || !w || !cu_seqlens) return GDN2_ERR_ARG;
  if (!workspace || !state_out || !o) return GDN2_ERR_ARG;
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return GDN2_ERR_ARG;
  if (nseq < 1 || T < 0 || H < 1 || HK < 1 || H % HK) return GDN2_ERR_ARG;
  if (DK != 64 && DK != 128) return GDN2_ERR_SHAPE;
  if (DV < 16 || DV % 16 || DV > 4096) return GDN2_ERR_SHAPE;
  if (T * H * DV * 4 >= (1L << 31)) return GDN2_ERR_SHAPE;   // 32-bit offsets in the DK = 128 scan
  const long slots = varlen_slots(nseq, T);
  if (static_cast<long>(HK) * slots > 0x7fffffffL || static_cast<long>(nseq) * H * (DV / 16) > 0x7fffffffL)
    return GDN2_ERR_SHAPE;
  const gdn2::Varlen vl{cu_seqlens, nseq};
  const hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned short* ws = static_cast<unsigned short*>(workspace);
  hipError_t e = gdn2::launch_chunk_local(q, k, b, g, in_dtype, 1, HK, DK, T, 0, static_cast<int>(slots),
                                          T, scale, ws, vl, st);
  if (e != hipSuccess) return status(e);
  return status(gdn2::launch_scan(v, w, in_dtype, ws, state_in, state_out, o, out_dtype, nseq, H, HK, DK,
                                  DV, T, 0, static_cast<int>(slots), T, vl, st));
}

static int layer_prologue(const void* xq, const void* xk, const void* xv, const void* xb,
                          const void* xw, const void* xf, long ld_q, long ld_k, long ld_v,
                          long ld_b, long ld_w, long ld_f, int act_dtype, const void* conv_w,
                          const void* conv_b, int conv_k, const void* conv_in, void* conv_out,
                          const float* a_log, const float* dt_bias, float erase_scale, void* q,
                          void* k, void* v, void* b, void* w, float* g, int B, long S, int H,
                          int HK, int DK, int DV, const int* cu_seqlens, int nseq, void* stream) {
  if (!dtype_ok(act_dtype) || B < 0 || S < 0 || H < 1 || HK < 1 || H % HK || DV < 1) return GDN2_ERR_ARG;
  // with no tokens nothing is read from the token buffers (they may be null);
  // only a packed batch's conv tails are written
  const bool tokens = static_cast<long>(B) * S > 0;
  if (tokens && (!xq || !xk || !xv || !xb || !xw || !xf || !a_log || !dt_bias)) return GDN2_ERR_ARG;
  if (tokens && (!q || !k || !v || !b || !w || !g)) return GDN2_ERR_ARG;
  const int dqk = HK * DK, dv = H * DV;
  if (ld_q < dqk || ld_k < dqk || ld_b < dqk || ld_f < dqk || ld_v < dv || ld_w < dv) return GDN2_ERR_ARG;
  // 8-channel lane items: DK / 8 lanes per q, k head, a power of two <= 64
  if (DK < 8 || DK % 8 || DK > 512 || ((DK / 8) & (DK / 8 - 1)) || DV % 8) return GDN2_ERR_SHAPE;
  // 16-byte vector accesses: rows and bases aligned
  const long lds[6] = {ld_q, ld_k, ld_v, ld_b, ld_w, ld_f};
  const void* xs[6] = {xq, xk, xv, xb, xw, xf};
  for (int i = 0; i < 6; ++i)
    if (lds[i] % 8 || (tokens && reinterpret_cast<uintptr_t>(xs[i]) % 16)) return GDN2_ERR_ARG;
  const void* outs[6] = {q, k, v, b, w, g};
  for (int i = 0; i < 6; ++i)
    if (tokens && reinterpret_cast<uintptr_t>(outs[i]) % 16) return GDN2_ERR_ARG;
  if (conv_w && (conv_k < 1 || conv_k > 4)) return GDN2_ERR_SHAPE;
  const void* cv[4] = {conv_w, conv_b, conv_in, conv_out};   // read / written as 16-byte vectors
  for (int i = 0; i < 4; ++i)
    if (conv_w && reinterpret_cast<uintptr_t>(cv[i]) % 16) return GDN2_ERR_ARG;
  if (conv_w && conv_out && conv_out == conv_in) return GDN2_ERR_ARG;   // the tail is read while written
  if (static_cast<long>(B) * S > 0x7fffffffL) return GDN2_ERR_SHAPE;
  gdn2::lay::ProArgs a;
  a.x[0] = xq; a.x[1] = xk; a.x[2] = xv; a.x[3] = xb; a.x[4] = xw; a.x[5] = xf;
  a.ld[0] = ld_q; a.ld[1] = ld_k; a.ld[2] = ld_v; a.ld[3] = ld_b; a.ld[4] = ld_w; a.ld[5] = ld_f;
  a.conv_w = conv_w; a.conv_b = conv_w ? conv_b : nullptr; a.K = conv_w ? conv_k : 0;
  a.conv_in = conv_w ? conv_in : nullptr; a.conv_out = conv_w ? conv_out : nullptr;
  a.a_log = a_log; a.dt_bias = dt_bias; a.erase_scale = erase_scale;
  a.q = q; a.k = k; a.v = v; a.b = b; a.w = w; a.g = g;
  a.B = B; a.S = S; a.H = H; a.HK = HK; a.DK = DK; a.DV = DV;
  a.cu = conv_w ? cu_seqlens : nullptr; a.nseq = nseq;
  return status(gdn2::launch_layer_prologue(a, act_dtype, static_cast<hipStream_t>(stream)));
}

int gdn2_hip_layer_prologue(const void* xq, const void* xk, const void* xv, const void* xb,
                            const void* xw, const void* xf, long ld_q, long ld_k, long ld_v,
                            long ld_b, long ld_w, long ld_f, int act_dtype, const void* conv_w,
                            const void* conv_b, int conv_k, const void* conv_in, void* conv_out,
                            const float* a_log, const float* dt_bias, float erase_scale, void* q,
                            void* k, void* v, void* b, void* w, float* g, int B, long S, int H,
                            int HK, int DK, int DV, void* stream) {
  return layer_prologue(xq, xk, xv, xb, xw, xf, ld_q, ld_k, ld_v, ld_b, ld_w, ld_f, act_dtype, conv_w, conv_b,
                        conv_k, conv_in, conv_out, a_log, dt_bias, erase_scale, q, k, v, b, w, g, B, S, H, HK, DK,
                        DV, nullptr, 0, stream);
}

int gdn2_hip_layer_prologue_varlen(const void* xq, const void* xk, const void* xv, const void* xb,
                                   const void* xw, const void* xf, long ld_q, long ld_k, long ld_v,
                                   long ld_b, long ld_w, long ld_f, int act_dtype, const void* conv_w,
                                   const void* conv_b, int conv_k, const void* conv_in, void* conv_out,
                                   const float* a_log, const float* dt_bias, float erase_scale, void* q, void* k,
                                   void* v, void* b, void* w, float* g, const int* cu_seqlens, int nseq, long T,
                                   int H, int HK, int DK, int DV, void* stream) {
  if (!cu_seqlens || nseq < 1) return GDN2_ERR_ARG;
  return layer_prologue(xq, xk, xv, xb, xw, xf, ld_q, ld_k, ld_v, ld_b, ld_w, ld_f, act_dtype, conv_w, conv_b,
                        conv_k, conv_in, conv_out, a_log, dt_bias, erase_scale, q, k, v, b, w, g, 1, T, H, HK, DK,
                        DV, cu_seqlens, nseq, stream);
}

int gdn2_hip_gemv(const void* x, long ldx, const void* W, void* y, long ldy, int dtype, int M, int N,
                  int K, void* stream) {
  if (!x || !W || !y) return GDN2_ERR_ARG;
  if (!dtype_ok(dtype) || M < 1 || N < 1 || K < 1 || ldx < K || ldy < N) return GDN2_ERR_ARG;
  if (M > 8 || K % 8) return GDN2_ERR_SHAPE;
  // 16-byte vector reads of x and W rows
  if (ldx % 8 || reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(W) % 16) return GDN2_ERR_ARG;
  return status(gdn2::launch_gemv(x, W, y, dtype, M, N, K, ldx, ldy, static_cast<hipStream_t>(stream)));
}

int gdn2_hip_layer_epilogue(const void* o, int o_dtype, const void* gate, long ld_gate,
                            const float* weight, float eps, void* out, int out_dtype, long ld_out,
                            int B, long S, int H, int DV, void* stream) {
  if (!o || !gate || !weight || !out) return GDN2_ERR_ARG;
  if (!dtype_ok(o_dtype) || !dtype_ok(out_dtype) || B < 0 || S < 0 || H < 1 || DV < 1) return GDN2_ERR_ARG;
  if (ld_gate < static_cast<long>(H) * DV || ld_out < static_cast<long>(H) * DV) return GDN2_ERR_ARG;
  const long rows = static_cast<long>(B) * S * H;
  if ((rows + 3) / 4 > 0x7fffffffL) return GDN2_ERR_SHAPE;
  return status(gdn2::launch_layer_epilogue(o, o_dtype, gate, ld_gate, weight, eps, out, out_dtype, ld_out,
                                            rows, H, DV, static_cast<hipStream_t>(stream)));
}

// Workspace of gdn2_hip_layer_decode: segments of M rows, each 256-byte aligned.
struct DecodeWs {
  size_t proj, q, k, b, v, w, g, o, normed, bytes;
};

static DecodeWs decode_ws(long M, int H, int HK, int DK, int DV, int dtype) {
  const size_t es = dtype == gdn2::DT_F32 ? 4 : 2;
  const long dqk = static_cast<long>(HK) * DK, dv = static_cast<long>(H) * DV;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  DecodeWs s;
  size_t at = 0;
  s.proj = at; at += up(M * (4 * dqk + 3 * dv) * es);
  s.q = at; at += up(M * dqk * es);
  s.k = at; at += up(M * dqk * es);
  s.b = at; at += up(M * dqk * es);
  s.v = at; at += up(M * dv * es);
  s.w = at; at += up(M * dv * es);
  s.g = at; at += up(M * dqk * 4);
  s.o = at; at += up(M * dv * es);
  s.normed = at; at += up(M * dv * es);
  s.bytes = at;
  return s;
}

size_t gdn2_hip_layer_decode_workspace_bytes(int B, int n, int H, int HK, int DK, int DV, int dtype) {
  if (B < 1 || n < 1 || H < 1 || HK < 1 || DK < 1 || DV < 1 || !dtype_ok(dtype)) return 0;
  return decode_ws(static_cast<long>(B) * n, H, HK, DK, DV, dtype).bytes;
}

int gdn2_hip_layer_decode(const void* x, const void* w_proj, const void* conv_w, const void* conv_b,
                          int conv_k, const void* conv_in, void* conv_out, const float* a_log,
                          const float* dt_bias, float erase_scale, float* state, const float* norm_w,
                          float norm_eps, const void* w_out, void* out, void* workspace, int dtype, int B,
                          int n, int hidden, int H, int HK, int DK, int DV, float scale, void* stream) {
  if (!x || !w_proj || !w_out || !out || !workspace || !state || !norm_w) return GDN2_ERR_ARG;
  if (B < 1 || n < 1 || hidden < 1 || H < 1 || HK < 1 || H % HK || !dtype_ok(dtype)) return GDN2_ERR_ARG;
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return GDN2_ERR_ARG;
  // Every stage's shape and alignment rule is checked before the first launch,
  // so the call either runs all of its launches or changes nothing.
  const long Ml = static_cast<long>(B) * n;
  if (Ml > 8) return GDN2_ERR_SHAPE;                                      // GEMV rows
  if (DK != 32 && DK != 64 && DK != 128 && DK != 256) return GDN2_ERR_SHAPE;   // decode
  if (DV % 32 || DV > 4096 || hidden % 8) return GDN2_ERR_SHAPE;           // decode, GEMV K
  const auto mis16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; };
  if (mis16(x) || mis16(w_proj) || mis16(w_out) || mis16(norm_w)) return GDN2_ERR_ARG;
  if (conv_w) {
    if (conv_k < 1 || conv_k > 4) return GDN2_ERR_SHAPE;
    if (mis16(conv_w) || mis16(conv_b) || mis16(conv_in) || mis16(conv_out)) return GDN2_ERR_ARG;
    if (conv_out && conv_out == conv_in) return GDN2_ERR_ARG;
  }
  if (!a_log || !dt_bias) return GDN2_ERR_ARG;
  const int M = static_cast<int>(Ml);
  const long dqk = static_cast<long>(HK) * DK, dv = static_cast<long>(H) * DV;
  const long ldp = 4 * dqk + 3 * dv;
  if (ldp > 0x7fffffffL) return GDN2_ERR_SHAPE;
  const DecodeWs s = decode_ws(M, H, HK, DK, DV, dtype);
  char* ws = static_cast<char*>(workspace);
  const size_t es = dtype == gdn2::DT_F32 ? 4 : 2;
  char* gate = ws + s.proj + (4 * dqk + 2 * dv) * es;   // o_gate rows, stride ldp
  const hipStream_t st = static_cast<hipStream_t>(stream);
  // 1. projections (one fused weight, rows q | k | v | b | w | f | o_gate)
  //    with conv + SiLU, gates and decay applied to the sums
  gdn2::gv::StepArgs a;
  a.x = x; a.W = w_proj; a.N = static_cast<int>(ldp); a.K = hidden; a.ldx = hidden;
  a.B = B; a.n = n; a.dqk = static_cast<int>(dqk); a.dv = static_cast<int>(dv); a.DK = DK;
  a.KC = conv_w ? conv_k : 0;
  a.conv_w = conv_w; a.conv_b = conv_w ? conv_b : nullptr;
  a.conv_in = conv_w ? conv_in : nullptr; a.conv_out = conv_w ? conv_out : nullptr;
  a.a_log = a_log; a.dt_bias = dt_bias; a.erase_scale = erase_scale;
  a.q = ws + s.q; a.k = ws + s.k; a.v = ws + s.v; a.b = ws + s.b; a.w = ws + s.w;
  a.g = reinterpret_cast<float*>(ws + s.g); a.gate = gate; a.ldg = ldp;
  if (hipError_t e = gdn2::launch_gemv_step(a, dtype, st)) return status(e);
  // 2. the recurrence, with the L2 norm of q and k in its staging pass
  if (hipError_t e = gdn2::launch_decode_layer(ws + s.q, ws + s.k, ws + s.v, reinterpret_cast<const float*>(ws + s.g),
                                               ws + s.b, ws + s.w, state, ws + s.o, B, H, HK, DK, DV, n, scale,
                                               dtype, st))
    return status(e);
  // 3. o_proj with the gated RMSNorm applied to its input on the fly
  if (gdn2::gemv_norm_supported(DV))
    return status(gdn2::launch_gemv_norm(ws + s.o, gate, ldp, norm_w, norm_eps, DV, w_out, out, dtype, M, hidden,
                                         static_cast<int>(dv), hidden, st));
  if (int e = gdn2_hip_layer_epilogue(ws + s.o, dtype, gate, ldp, norm_w, norm_eps, ws + s.normed, dtype, dv, B,
                                      n, H, DV, stream))
    return e;
  return gdn2_hip_gemv(ws + s.normed, dv, w_out, out, hidden, dtype, M, hidden, static_cast<int>(dv), stream);
}

static int backward_shape(int B, long S, int H, int HK, int DK, int DV) {
  if (B < 1 || S < 0 || H < 1 || HK < 1 || H % HK) return GDN2_ERR_ARG;
  if (DK != 32 && DK != 64 && DK != 128) return GDN2_ERR_SHAPE;
  if (DV < 16 || DV % 16 || DV > 4096) return GDN2_ERR_SHAPE;
  const long NC = (S + gdn2::kBS - 1) / gdn2::kBS;
  // grid dimensions and 32-bit element counts of the fp32 intermediates
  if (NC > 65535 || static_cast<long>(B) * H > 65535) return GDN2_ERR_SHAPE;
  if (NC * (DK / 32) * B * H > 0x7fffffffL) return GDN2_ERR_SHAPE;   // pairwise pass: one-dimensional grid
  if (static_cast<long>(B) * S * HK * DK > 0x7fffffffL) return GDN2_ERR_SHAPE;
  return 0;
}

size_t gdn2_hip_backward_workspace_bytes(int B, int H, int HK, int DK, int DV, long S) {
  if (backward_shape(B, S, H, HK, DK, DV)) return 0;
  return gdn2::backward_workspace_bytes(B, H, HK, DK, DV, S);
}

int gdn2_hip_backward(const void* q, const void* k, const void* v, const float* g, const void* b, const void* w,
                      int in_dtype, float scale, const float* initial_state, const void* d_out, int do_dtype,
                      const float* d_final_state, void* dq, void* dk, void* dv, float* dg, void* db, void* dw,
                      float* d_initial_state, void* workspace, int B, long S, int H, int HK, int DK, int DV,
                      void* stream) {
  if (!dtype_ok(in_dtype) || !dtype_ok(do_dtype)) return GDN2_ERR_ARG;
  if (int e = backward_shape(B, S, H, HK, DK, DV)) return e;
  if (S > 0 && (!q || !k || !v || !g || !b || !w || !d_out || !dq || !dk || !dv || !dg || !db || !dw || !workspace))
    return GDN2_ERR_ARG;
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return GDN2_ERR_ARG;
  return status(gdn2::launch_backward(q, k, v, g, b, w, in_dtype, scale, initial_state, d_out, do_dtype,
                                      d_final_state, dq, dk, dv, dg, db, dw, d_initial_state, workspace, B, H, HK,
                                      DK, DV, S, static_cast<hipStream_t>(stream)));
}

static int backward_varlen_shape(int nseq, long T, int H, int HK, int DK, int DV) {
  if (nseq < 1 || T < 0 || H < 1 || HK < 1 || H % HK) return GDN2_ERR_ARG;
  if (DK != 32 && DK != 64 && DK != 128) return GDN2_ERR_SHAPE;
  if (DV < 16 || DV % 16 || DV > 4096) return GDN2_ERR_SHAPE;
  const long NC = varlen_slots(nseq, T);
  if (NC > 0x7fffffffL / 4 || H > 65535) return GDN2_ERR_SHAPE;
  if (NC * (DK / 32) * H > 0x7fffffffL) return GDN2_ERR_SHAPE;   // pairwise pass: one-dimensional grid
  if (static_cast<long>(nseq) * H * (DV / 16) * 2 > 0x7fffffffL) return GDN2_ERR_SHAPE;   // scan grid
  if (T * HK * DK > 0x7fffffffL) return GDN2_ERR_SHAPE;
  return 0;
}

size_t gdn2_hip_backward_varlen_workspace_bytes(int nseq, int H, int HK, int DK, int DV, long T) {
  if (backward_varlen_shape(nseq, T, H, HK, DK, DV)) return 0;
  return gdn2::backward_varlen_workspace_bytes(nseq, H, HK, DK, DV, T);
}

int gdn2_hip_backward_varlen(const void* q, const void* k, const void* v, const float* g, const void* b,
                             const void* w, int in_dtype, float scale, const float* initial_state,
                             const void* d_out, int do_dtype, const float* d_final_state, void* dq, void* dk,
                             void* dv, float* dg, void* db, void* dw, float* d_initial_state, void* workspace,
                             const int* cu_seqlens, int nseq, long T, int H, int HK, int DK, int DV,
                             void* stream) {
  if (!dtype_ok(in_dtype) || !dtype_ok(do_dtype)) return GDN2_ERR_ARG;
  if (int e = backward_varlen_shape(nseq, T, H, HK, DK, DV)) return e;
  if (!cu_seqlens) return GDN2_ERR_ARG;
  if (T > 0 && (!q || !k || !v || !g || !b || !w || !d_out || !dq || !dk || !dv || !dg || !db || !dw || !workspace))
    return GDN2_ERR_ARG;
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return GDN2_ERR_ARG;
  return status(gdn2::launch_backward_varlen(q, k, v, g, b, w, in_dtype, scale, initial_state, d_out, do_dtype,
                                             d_final_state, dq, dk, dv, dg, db, dw, d_initial_state, workspace,
                                             cu_seqlens, nseq, H, HK, DK, DV, T, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
