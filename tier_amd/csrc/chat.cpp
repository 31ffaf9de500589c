// chat.cpp -- the chat engine's linear-layer dispatch with weight streaming.
//
// chat_lin (tier.cpp:2351-2378) runs one linear y = x * W^T of a decoder layer:
// quantized rows go to gemv_q at M = 1 and to dequant + GEMM above, fp16 / bf16
// rows to gemv<T> or the x3 products (chat_fp3 / chat_bf3).  Matrices that do
// not fit in device memory stay in pinned host memory and are streamed through
// a ring of device slots (g_chat_SQ, chat_slot, chat_issue, tier.cpp:2283-2285):
// each streamed matrix is used in a fixed cyclic order; the copy of use i goes
// into slot i % nslots on a copy stream after use i - nslots released that slot,
// and use i waits for its copy on the compute stream.  Placement follows the
// engine's rule (tier.cpp:2549-2555): in registration order a matrix stays
// resident while it fits beside the reserve, and every matrix after the first
// one that does not fit is streamed.
//
// After the base product a matrix may get the engine's two additions: trained
// rows written over their rows of the output (chat_heads, tier.cpp:2339-2350)
// and a LoRA adapter's s * (x A^T) B^T (chat_lora, tier.cpp:2333-2337).
//
// Differences from the engine, on purpose: the number of slots is a parameter
// (2 in the engine); a streamed matrix used out of the cyclic order is refused
// instead of computing with another matrix's rows; streamed host memory must be
// pinned (a pageable copy would serialise the host with the copy).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <vector>

#include "tm_host.h"

namespace tiermm {
bool gpu_type(int qtype);
int chat_scatter_cols(const float* src, float* y, const int* idx, int M, int r, int ld, hipStream_t s);
int chat_scale(float* u, size_t n, float f, hipStream_t s);
}

using namespace tiermm;

struct tiermm_chat {
  struct Mat {
    int qtype;
    size_t rb;
    int rows, cols;
    size_t bytes;
    const void* host;  // host rows (the streaming source), may be null for caller-resident rows
    void* dev;         // device rows; null while the matrix is streamed or not yet placed
    bool owned;        // dev was allocated by tiermm_chat_place
    // trained rows (chat_heads, tier.cpp:2339-2350): hr rows of htype at hd replace
    // output rows ri[j] (rows 0..hr-1 without ri); caller-owned device memory
    int hr = 0, htype = 0;
    const void* hd = nullptr;
    const int* ri = nullptr;
    // LoRA adapter (chat_lora, tier.cpp:2333-2337): y += s * (x A^T) B^T, A [lr][cols],
    // B [rows][lr] fp32, caller-owned device memory
    int lr = 0;
    const float* la = nullptr;
    const float* lb = nullptr;
  };
  int device = 0;
  int nslots = 2;
  hipStream_t cs = nullptr;  // compute stream (the caller's)
  hipStream_t ms = nullptr;  // copy stream (owned)
  std::vector<Mat> mats;
  std::vector<int> sq;  // streamed matrices in use order
  std::vector<void*> slot;
  std::vector<hipEvent_t> ev_cp, ev_done;
  long long qi = 0;  // uses of streamed matrices so far
  bool placed = false;
  size_t resident = 0, streamed = 0;
  bool heads_on = true;                   // g_chat_heads (tier.cpp:2338)
  float lora_alpha = 0.f, lora_k = 1.f;   // g_chat_lalpha, g_chat_lk (tier.cpp:2332)
  bool lora_on = true;                    // g_chat_lon
  float* htmp = nullptr;                  // trained rows' outputs before the scatter
  size_t htmp_n = 0;
  float* lu = nullptr;                    // x A^T of the LoRA adapter
  size_t lu_n = 0;
};

namespace {

bool dense(int t) { return t == QT_F32 || t == QT_F16 || t == QT_BF16; }

int on_device(const tiermm_chat* c, const char* who) {
  int d = -1;
  hipError_t e = hipGetDevice(&d);
  if (e != hipSuccess) return hip_fail(e, who);
  if (d != c->device) return set_error(TIERMM_EINVAL, "%s: device %d is current, the set lives on %d", who, d, c->device);
  return TIERMM_OK;
}

// chat_issue (tier.cpp:2285): copy the matrix of use i into slot i % nslots
// once use i - nslots has released it.
int issue(tiermm_chat* c, long long i) {
  const int s = (int)(i % c->nslots);
  const auto& m = c->mats[(size_t)c->sq[(size_t)(i % (long long)c->sq.size())]];
  hipError_t e = hipStreamWaitEvent(c->ms, c->ev_done[s], 0);
  if (e == hipSuccess && m.bytes) e = hipMemcpyAsync(c->slot[s], m.host, m.bytes, hipMemcpyHostToDevice, c->ms);
  if (e == hipSuccess) e = hipEventRecord(c->ev_cp[s], c->ms);
  return e == hipSuccess ? TIERMM_OK : hip_fail(e, "tiermm_chat: weight copy");
}

bool pinned(const void* p) {
  hipPointerAttribute_t a;
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();  // pageable memory is reported as an error by some runtimes
    return false;
  }
  return a.type == hipMemoryTypeHost;
}

void release(tiermm_chat* c) {
  if (c->ms) (void)hipStreamSynchronize(c->ms);
  if (c->placed) (void)hipStreamSynchronize(c->cs);
  for (auto& m : c->mats)
    if (m.owned && m.dev) (void)hipFree(m.dev);
  for (void* p : c->slot)
    if (p) (void)hipFree(p);
  if (c->htmp) (void)hipFree(c->htmp);
  if (c->lu) (void)hipFree(c->lu);
  for (auto e : c->ev_cp)
    if (e) (void)hipEventDestroy(e);
  for (auto e : c->ev_done)
    if (e) (void)hipEventDestroy(e);
  if (c->ms) (void)hipStreamDestroy(c->ms);
  delete c;
}

// The product of one linear, as chat_lin chooses it.
int compute(const tiermm_chat::Mat& m, const void* W, const float* x, float* y, int M, int mode, hipStream_t s) {
  const tiermm_stream_t st = (tiermm_stream_t)s;
  if (M == 1)  // gemv<T> (tier.cpp:2363) / gemv_q (tier.cpp:2357)
    return dense(m.qtype) ? tiermm_gemv(W, m.qtype, x, y, m.rows, m.cols, st)
                          : tiermm_qgemv(W, m.qtype, m.rb, x, y, m.rows, m.cols, st);
  if (m.qtype == QT_F16 && mode == TIERMM_MODE_X3REF) {  // chat_fp3 (tier.cpp:2368)
    const int r = tiermm_x3_rows((const uint16_t*)W, x, y, M, m.cols, m.rows, m.rows, nullptr, 0, st);
    if (r != TIERMM_UNSUPPORTED) return r;
  } else if (m.qtype == QT_BF16 && mode == TIERMM_MODE_X3REF) {  // chat_bf3 (tier.cpp:2370)
    const int r = tiermm_x3_rows_bf16((const uint16_t*)W, x, y, M, m.cols, m.rows, m.rows, nullptr, 0, st);
    if (r != TIERMM_UNSUPPORTED) return r;
  }
  // quantized prefill (dequant + GEMM, tier.cpp:2358-2359), fp32 rows (chat_linear), and the
  // fp32 fallback of the dense types (expand + SGEMM, tier.cpp:2372-2374)
  const int md = dense(m.qtype) ? TIERMM_MODE_F32 : mode;
  return tiermm_qgemm(W, m.qtype, m.rb, x, y, M, m.rows, m.cols, m.rows, md, 0.f, nullptr, 0, st);
}

// A float buffer of at least n elements on the set's device, grown as the
// engine's g_chat_htmp / g_chat_lu are (tier.cpp:2335, 2341); the old one may
// still be read by queued work, so the stream is drained before it is freed.
int grow(tiermm_chat* c, float*& buf, size_t& have, size_t n, const char* who) {
  if (n <= have) return TIERMM_OK;
  hipError_t e = hipSuccess;
  if (buf) {
    e = hipStreamSynchronize(c->cs);
    if (e == hipSuccess) e = hipFree(buf);
    buf = nullptr;
    have = 0;
    if (e != hipSuccess) return hip_fail(e, who);
  }
  e = hipMalloc(&buf, n * sizeof(float));
  if (e != hipSuccess) {
    buf = nullptr;
    return hip_fail(e, who);
  }
  have = n;
  return TIERMM_OK;
}

// chat_heads (tier.cpp:2339-2350): the trained rows' product -- gemv<T> at M = 1,
// the fp32 expand + SGEMM semantics above -- written over their rows of y.
int apply_heads(tiermm_chat* c, const tiermm_chat::Mat& m, const float* x, float* y, int M) {
  const char* who = "tiermm_chat_lin: trained rows";
  const tiermm_stream_t st = (tiermm_stream_t)c->cs;
  float* dst = y;
  int ld = m.rows;
  if (m.ri) {
    const int r = grow(c, c->htmp, c->htmp_n, (size_t)M * m.hr, who);
    if (r) return r;
    dst = c->htmp;
    ld = m.hr;
  }
  int r = M == 1 ? tiermm_gemv(m.hd, m.htype, x, dst, m.hr, m.cols, st)
                 : tiermm_qgemm(m.hd, m.htype, (size_t)m.cols * 2, x, dst, M, m.hr, m.cols, ld, TIERMM_MODE_F32, 0.f,
                                nullptr, 0, st);
  if (r || !m.ri) return r;
  return chat_scatter_cols(c->htmp, y, m.ri, M, m.hr, m.rows, c->cs);
}

// chat_lora (tier.cpp:2333-2337): y += s * (x A^T) B^T with s = k * alpha / r while the
// adapter is on (0 skips it), both products fp32-accurate (TIERMM_MODE_F32).
int apply_lora(tiermm_chat* c, const tiermm_chat::Mat& m, const float* x, float* y, int M) {
  const float s = c->lora_on ? c->lora_k * c->lora_alpha / (float)m.lr : 0.f;
  if (s == 0.f) return TIERMM_OK;
  const char* who = "tiermm_chat_lin: lora";
  const tiermm_stream_t st = (tiermm_stream_t)c->cs;
  int r = grow(c, c->lu, c->lu_n, (size_t)M * m.lr, who);
  if (!r) r = tiermm_qgemm(m.la, QT_F32, (size_t)m.cols * 4, x, c->lu, M, m.lr, m.cols, m.lr, TIERMM_MODE_F32, 0.f,
                           nullptr, 0, st);
  if (!r) r = chat_scale(c->lu, (size_t)M * m.lr, s, c->cs);
  if (!r) r = tiermm_qgemm(m.lb, QT_F32, (size_t)m.lr * 4, c->lu, y, M, m.rows, m.lr, m.rows, TIERMM_MODE_F32, 1.f,
                           nullptr, 0, st);
  return r;
}

}  // namespace

extern "C" {

int tiermm_chat_create(int nslots, tiermm_stream_t compute_stream, tiermm_chat** out) {
  if (!out) return set_error(TIERMM_EINVAL, "tiermm_chat_create: null output");
  *out = nullptr;
  if (nslots < 2 || nslots > 8) return set_error(TIERMM_EINVAL, "tiermm_chat_create: %d slots (2..8)", nslots);
  auto* c = new tiermm_chat;
  c->nslots = nslots;
  c->cs = (hipStream_t)compute_stream;
  hipError_t e = hipGetDevice(&c->device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->ms, hipStreamNonBlocking);
  c->ev_cp.assign(nslots, nullptr);
  c->ev_done.assign(nslots, nullptr);
  for (int i = 0; e == hipSuccess && i < nslots; ++i) {
    e = hipEventCreateWithFlags(&c->ev_cp[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->ev_done[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(c->ev_done[i], c->cs);  // every slot starts free
  }
  if (e != hipSuccess) {
    const int r = hip_fail(e, "tiermm_chat_create");
    release(c);
    return r;
  }
  *out = c;
  return TIERMM_OK;
}

void tiermm_chat_destroy(tiermm_chat* c) {
  if (c) release(c);
}

int tiermm_chat_add(tiermm_chat* c, int qtype, size_t rb, int rows, int cols, const void* host, void* dev, int* id) {
  const char* who = "tiermm_chat_add";
  if (!c || !id) return set_error(TIERMM_EINVAL, "%s: null argument", who);
  if (c->placed) return set_error(TIERMM_EINVAL, "%s: matrices are added before tiermm_chat_place", who);
  const BlockInfo* b = block_info(qtype);
  if (!b || !gpu_type(qtype)) return set_error(TIERMM_UNSUPPORTED, "%s: type %d is not handled on the GPU", who, qtype);
  const int whole = std::max(8, b->elems);
  if (rows <= 0 || cols <= 0 || cols % whole)
    return set_error(TIERMM_EINVAL, "%s: %d x %d %s (columns in whole blocks of %d)", who, rows, cols, b->name, whole);
  if (rb != (size_t)(cols / b->elems) * b->bytes)
    return set_error(TIERMM_EINVAL, "%s: rb %zu does not match %d %s columns", who, rb, cols, b->name);
  if (!host && !dev) return set_error(TIERMM_EINVAL, "%s: neither host nor device rows", who);
  if (dev && ((uintptr_t)dev % 16)) return set_error(TIERMM_EINVAL, "%s: device rows must be 16-byte aligned", who);
  tiermm_chat::Mat m{qtype, rb, rows, cols, rb * (size_t)rows, host, dev, false};
  *id = (int)c->mats.size();
  c->mats.push_back(m);
  return TIERMM_OK;
}

int tiermm_chat_place(tiermm_chat* c, size_t budget, size_t reserve, size_t* resident_bytes,
                      size_t* streamed_bytes) {
  const char* who = "tiermm_chat_place";
  if (!c) return set_error(TIERMM_EINVAL, "%s: null set", who);
  if (c->placed) return set_error(TIERMM_EINVAL, "%s: the set is placed already", who);
  int st = on_device(c, who);
  if (st) return st;
  size_t fr = 0, tt = 0;
  hipError_t e = hipMemGetInfo(&fr, &tt);
  if (e != hipSuccess) return hip_fail(e, who);
  // the slots are sized for the largest matrix still to place, as the engine's
  // chat_slot are allocated before the placement
  size_t maxmb = 0;
  for (const auto& m : c->mats)
    if (!m.dev) maxmb = std::max(maxmb, m.bytes);
  const size_t slots = (size_t)c->nslots * ((maxmb + 255) & ~(size_t)255);
  const size_t avail = fr > slots ? fr - slots : 0;
  auto undo = [c](int code) {  // leave the set as it was before the call
    for (auto& m : c->mats)
      if (m.owned) {
        (void)hipFree(m.dev);
        m.dev = nullptr;
        m.owned = false;
      }
    for (void* p : c->slot)
      if (p) (void)hipFree(p);
    c->slot.clear();
    c->sq.clear();
    c->resident = c->streamed = 0;
    return code;
  };
  size_t used = 0;
  bool full = false;
  for (size_t i = 0; i < c->mats.size(); ++i) {
    auto& m = c->mats[i];
    if (m.dev) continue;  // resident in the caller's memory
    bool fit = !full && used + m.bytes <= budget && used + m.bytes + reserve < avail;
    if (fit && hipMalloc(&m.dev, std::max<size_t>(m.bytes, 1)) != hipSuccess) {
      (void)hipGetLastError();
      m.dev = nullptr;
      fit = false;
    }
    if (fit) {
      m.owned = true;
      e = hipMemcpy(m.dev, m.host, m.bytes, hipMemcpyHostToDevice);
      if (e != hipSuccess) return undo(hip_fail(e, who));
      used += m.bytes;
      continue;
    }
    full = true;
    if (!pinned(m.host))
      return undo(set_error(TIERMM_EINVAL,
                            "%s: matrix %zu is streamed but its host rows are not pinned (tiermm_host_alloc)", who, i));
    c->sq.push_back((int)i);
    c->streamed += m.bytes;
  }
  c->resident = used;
  if (!c->sq.empty()) {
    size_t sb = 0;
    for (int i : c->sq) sb = std::max(sb, c->mats[(size_t)i].bytes);
    c->slot.assign(c->nslots, nullptr);
    for (int s = 0; s < c->nslots; ++s) {
      e = hipMalloc(&c->slot[s], std::max<size_t>(sb, 1));
      if (e != hipSuccess) {
        c->slot[s] = nullptr;
        return undo(hip_fail(e, "tiermm_chat_place: slot"));
      }
    }
    for (int i = 0; i < c->nslots; ++i) {  // the first copies (tier.cpp:2569)
      st = issue(c, i);
      if (st) {
        (void)hipStreamSynchronize(c->ms);
        return undo(st);
      }
    }
  }
  c->placed = true;
  if (resident_bytes) *resident_bytes = c->resident;
  if (streamed_bytes) *streamed_bytes = c->streamed;
  return TIERMM_OK;
}

int tiermm_chat_lin(tiermm_chat* c, int id, const float* x, float* y, int M, int mode) {
  const char* who = "tiermm_chat_lin";
  if (!c) return set_error(TIERMM_EINVAL, "%s: null set", who);
  if (id < 0 || id >= (int)c->mats.size()) return set_error(TIERMM_EINVAL, "%s: matrix %d of %zu", who, id, c->mats.size());
  if (M < 1 || !x || !y) return set_error(TIERMM_EINVAL, "%s: M=%d, x and y device rows", who, M);
  if (mode != TIERMM_MODE_X3REF && mode != TIERMM_MODE_F32) return set_error(TIERMM_EINVAL, "%s: mode %d", who, mode);
  const auto& m = c->mats[(size_t)id];
  if (!m.dev && !c->placed) return set_error(TIERMM_EINVAL, "%s: matrix %d is not placed (tiermm_chat_place)", who, id);
  int st = on_device(c, who);
  if (st) return st;
  const void* W = m.dev;
  long long my = -1;
  if (!W) {
    const int next = c->sq[(size_t)(c->qi % (long long)c->sq.size())];
    if (next != id)
      return set_error(TIERMM_EINVAL, "%s: streamed matrix %d used out of order, matrix %d is next (tiermm_chat_restart)",
                       who, id, next);
    my = c->qi++;
    hipError_t e = hipStreamWaitEvent(c->cs, c->ev_cp[(size_t)(my % c->nslots)], 0);
    if (e != hipSuccess) return hip_fail(e, who);
    W = c->slot[(size_t)(my % c->nslots)];
  }
  st = compute(m, W, x, y, M, mode, c->cs);
  if (!st && m.hr && c->heads_on) st = apply_heads(c, m, x, y, M);  // tier.cpp:2375
  if (!st && m.lr) st = apply_lora(c, m, x, y, M);                   // tier.cpp:2376
  if (my >= 0) {  // release the slot and refill it with the use nslots ahead (tier.cpp:2377)
    hipError_t e = hipEventRecord(c->ev_done[(size_t)(my % c->nslots)], c->cs);
    const int r = e == hipSuccess ? issue(c, my + c->nslots) : hip_fail(e, who);
    if (!st) st = r;
  }
  return st;
}

int tiermm_chat_restart(tiermm_chat* c, int rewind) {
  if (!c) return set_error(TIERMM_EINVAL, "tiermm_chat_restart: null set");
  if (!c->placed || c->sq.empty()) return TIERMM_OK;
  hipError_t e = hipStreamSynchronize(c->cs);
  if (e == hipSuccess) e = hipStreamSynchronize(c->ms);
  if (e != hipSuccess) return hip_fail(e, "tiermm_chat_restart");
  if (rewind) c->qi = 0;
  for (int j = 0; j < c->nslots; ++j) {  // the engine's chat_issue(qi), chat_issue(qi+1) after a weight change
    const int st = issue(c, c->qi + j);
    if (st) return st;
  }
  return TIERMM_OK;
}

int tiermm_chat_info(const tiermm_chat* c, int id, int* streamed, size_t* resident_bytes, size_t* streamed_bytes,
                     long long* uses) {
  if (!c) return set_error(TIERMM_EINVAL, "tiermm_chat_info: null set");
  if (id >= (int)c->mats.size()) return set_error(TIERMM_EINVAL, "tiermm_chat_info: matrix %d", id);
  if (streamed) *streamed = id >= 0 ? (c->placed && !c->mats[(size_t)id].dev) : -1;
  if (resident_bytes) *resident_bytes = c->resident;
  if (streamed_bytes) *streamed_bytes = c->streamed;
  if (uses) *uses = c->qi;
  return TIERMM_OK;
}

int tiermm_chat_set_heads(tiermm_chat* c, int id, int hr, int htype, const void* hd, const int* ri) {
  const char* who = "tiermm_chat_set_heads";
  if (!c || id < 0 || id >= (int)c->mats.size()) return set_error(TIERMM_EINVAL, "%s: matrix %d", who, id);
  auto& m = c->mats[(size_t)id];
  if (hr == 0 || !hd) {
    m.hr = 0;
    m.hd = nullptr;
    m.ri = nullptr;
    return TIERMM_OK;
  }
  if (hr < 0 || hr > m.rows) return set_error(TIERMM_EINVAL, "%s: %d rows of %d", who, hr, m.rows);
  if (htype != QT_F16 && htype != QT_BF16) return set_error(TIERMM_EINVAL, "%s: row type %d (F16 or BF16)", who, htype);
  if ((uintptr_t)hd % 16) return set_error(TIERMM_EINVAL, "%s: rows must be 16-byte aligned", who);
  m.hr = hr;
  m.htype = htype;
  m.hd = hd;
  m.ri = ri;
  return TIERMM_OK;
}

int tiermm_chat_heads(tiermm_chat* c, int on) {
  if (!c) return set_error(TIERMM_EINVAL, "tiermm_chat_heads: null set");
  c->heads_on = on != 0;
  return TIERMM_OK;
}

int tiermm_chat_set_lora(tiermm_chat* c, int id, int r, const float* A, const float* B) {
  const char* who = "tiermm_chat_set_lora";
  if (!c || id < 0 || id >= (int)c->mats.size()) return set_error(TIERMM_EINVAL, "%s: matrix %d", who, id);
  auto& m = c->mats[(size_t)id];
  if (r == 0 || !A || !B) {
    m.lr = 0;
    m.la = m.lb = nullptr;
    return TIERMM_OK;
  }
  if (r < 0) return set_error(TIERMM_EINVAL, "%s: rank %d", who, r);
  if (((uintptr_t)A | (uintptr_t)B) % 4) return set_error(TIERMM_EINVAL, "%s: A and B must be 4-byte aligned", who);
  m.lr = r;
  m.la = A;
  m.lb = B;
  return TIERMM_OK;
}

int tiermm_chat_lora_scale(tiermm_chat* c, float alpha, float k, int on) {
  if (!c) return set_error(TIERMM_EINVAL, "tiermm_chat_lora_scale: null set");
  c->lora_alpha = alpha;
  c->lora_k = k;
  c->lora_on = on != 0;
  return TIERMM_OK;
}

int tiermm_host_alloc(size_t bytes, void** out) {
  if (!out) return set_error(TIERMM_EINVAL, "tiermm_host_alloc: null output");
  *out = nullptr;
  hipError_t e = hipHostMalloc(out, std::max<size_t>(bytes, 1), hipHostMallocDefault);
  if (e != hipSuccess) {
    *out = nullptr;
    return hip_fail(e, "tiermm_host_alloc");
  }
  return TIERMM_OK;
}

int tiermm_host_free(void* p) {
  if (!p) return TIERMM_OK;
  hipError_t e = hipHostFree(p);
  return e == hipSuccess ? TIERMM_OK : hip_fail(e, "tiermm_host_free");
}

}  // extern "C"
