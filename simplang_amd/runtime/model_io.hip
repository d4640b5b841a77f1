// model_io.hip -- model files around the decode path: the llama2.c checkpoint
// and tokenizer the reference host reads, the reference's temperature sampler,
// W4 quantizers on the GPU, and a packed W4 (symmetric) model file.
//
// Reference behaviour restated:
//   checkpoint  examples/llama2/generate_stories110M.cpp:143-191: a 7-int32
//               llama2.c Config header, then fp32 tensors in the order
//               token_embedding, rms_att, wq, wk, wv, wo, rms_ffn, w1, w2, w3,
//               rms_final, [wcls]; vocab_size > 0 means the classifier shares
//               the embedding table.  (The reference sizes wk/wv as dim x dim
//               and reads wcls right after rms_final; llama2.c's own layout
//               sizes them kv_dim x dim and has 2 * seq_len * head_size/2
//               floats of legacy RoPE tables before wcls.  The two agree for
//               the checkpoints the reference runs: n_kv_heads == n_heads and
//               a shared classifier.  Here the llama2.c layout is read, so
//               grouped-query and unshared checkpoints load correctly too.)
//   tokenizer   generate_stories110M.cpp:36-70: int32 max_token_length, then per
//               token a float score, an int32 length and the bytes; decode()
//               returns the token's bytes, "?" when out of range.
//   sampling    generate_stories110M.cpp:73-116: argmax with strict '>' from
//               index 0 for temperature 0; otherwise logits / T, softmax with
//               the max subtracted, one std::uniform_real_distribution<float>
//               draw from a std::mt19937, the first i with r < cdf_i (else the
//               last index).
//   W4 (ref.)   examples/llama2/bench_llama_quant.cpp:51-93 quantize_w4: flat
//               groups of `gs` over a tensor, scale = (max - min) / 15 (at
//               least 1e-8), zero = min, q = clamp(round((w - min) / scale),
//               0, 15), low nibble = even index.
//   W4 (sym.)   the benchmark W4 format: per row, groups of gs along K, scale =
//               max|w| / 7 (1 for an all-zero group), q = clamp(round(w / s),
//               -8, 7).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "rt_device.h"
#include "rt_internal.h"

namespace simp {
namespace {

// One wave per group: min/max over the group, then each lane quantizes and
// packs pairs of elements.  Groups are flat runs over the tensor (the last may
// be short); the tensor's nibbles start at byte 0 of q, as each tensor's do in
// the reference (quantize_w4 appends every tensor at a byte boundary).
__global__ void __launch_bounds__(256)
    quant_w4u_k(const float *__restrict__ w, int64_t n, int gs, uint8_t *__restrict__ q,
                float *__restrict__ scales, float *__restrict__ zeros) {
  const int lane = threadIdx.x & 63;
  const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t ngroups = (n + gs - 1) / gs;
  if (g >= ngroups) return;
  const int64_t start = g * gs, end = min(start + (int64_t)gs, n);
  float mn = w[start], mx = w[start];
  for (int64_t i = start + lane; i < end; i += 64) {
    mn = fminf(mn, w[i]);
    mx = fmaxf(mx, w[i]);
  }
  for (int d = 32; d >= 1; d >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, d));
    mx = fmaxf(mx, __shfl_xor(mx, d));
  }
  float scale = (mx - mn) / 15.0f;
  if (scale < 1e-8f) scale = 1e-8f;
  if (lane == 0) {
    scales[g] = scale;
    zeros[g] = mn;
  }
  // byte b holds elements 2b (low nibble) and 2b+1; gs is even, so a group
  // owns whole bytes (a short last group of odd length leaves its last high
  // nibble zero, as the reference's zero-initialised vector does)
  for (int64_t i = start + 2 * lane; i < end; i += 128) {
    uint32_t b = (uint32_t)max(0, min(15, (int)roundf((w[i] - mn) / scale)));
    if (i + 1 < end) b |= (uint32_t)max(0, min(15, (int)roundf((w[i + 1] - mn) / scale))) << 4;
    q[i >> 1] = (uint8_t)b;
  }
}

// Symmetric: one wave per (row, group).
__global__ void __launch_bounds__(256)
    quant_w4s_k(const float *__restrict__ w, int64_t rows, int64_t cols, int gs,
                uint8_t *__restrict__ q, float *__restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int64_t gpr = cols / gs;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= rows * gpr) return;
  const int64_t r = t / gpr, g = t - r * gpr;
  const float *src = w + r * cols + g * gs;
  float amax = 0.f;
  for (int i = lane; i < gs; i += 64) amax = fmaxf(amax, fabsf(src[i]));
  for (int d = 32; d >= 1; d >>= 1) amax = fmaxf(amax, __shfl_xor(amax, d));
  const float s = amax > 0.f ? amax / 7.0f : 1.0f;
  if (lane == 0) scales[r * gpr + g] = s;
  uint8_t *dst = q + r * (cols / 2) + g * (gs / 2);
  for (int i = 2 * lane; i < gs; i += 128) {
    const int a = max(-8, min(7, (int)roundf(src[i] / s)));
    const int b = max(-8, min(7, (int)roundf(src[i + 1] / s)));
    dst[i >> 1] = (uint8_t)((a & 15) | ((b & 15) << 4));
  }
}

// Reads `bytes` from f into device memory at dst through a pinned staging
// buffer, copies overlapped with the next read.
int read_to_device(FILE *f, void *dst, size_t bytes, hipStream_t st, const char *what) {
  constexpr size_t kChunk = 32u << 20;
  void *stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int rc = SIMP_RT_OK;
  for (int i = 0; i < 2; i++) {
    if (hipHostMalloc(&stage[i], kChunk, hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&done[i], hipEventDisableTiming) != hipSuccess) {
      rc = set_error(SIMP_RT_ENOMEM, "%s: pinned staging buffers", what);
      break;
    }
  }
  size_t off = 0;
  int b = 0;
  while (rc == SIMP_RT_OK && off < bytes) {
    const size_t n = std::min(kChunk, bytes - off);
    if (hipEventSynchronize(done[b]) != hipSuccess) {  // the copy from this buffer ended
      rc = set_error(SIMP_RT_EHIP, "%s: staging copy", what);
      break;
    }
    if (fread(stage[b], 1, n, f) != n) {
      rc = set_error(SIMP_RT_EINVAL, "%s: file ends before byte %zu of %zu", what, off + n, bytes);
      break;
    }
    if (hipMemcpyAsync((char *)dst + off, stage[b], n, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipEventRecord(done[b], st) != hipSuccess) {
      rc = set_error(SIMP_RT_EHIP, "%s: staging copy", what);
      break;
    }
    off += n;
    b ^= 1;
  }
  if (hipStreamSynchronize(st) != hipSuccess && rc == SIMP_RT_OK)
    rc = set_error(SIMP_RT_EHIP, "%s: staging copy", what);
  for (int i = 0; i < 2; i++) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (stage[i]) (void)hipHostFree(stage[i]);
  }
  return rc;
}

struct FileCloser {
  FILE *f;
  ~FileCloser() {
    if (f) fclose(f);
  }
};

// Tensor sizes (in floats) of a llama2.c checkpoint, in file order.
struct CkptLayout {
  int64_t emb, rms_att, wq, wk, wv, wo, rms_ffn, w1, w2, w3, rms_final, freq, wcls;
  bool shared;
  int64_t total() const {
    return emb + rms_att + wq + wk + wv + wo + rms_ffn + w1 + w2 + w3 + rms_final + freq + wcls;
  }
};

int ckpt_layout(const simp_rt_ckpt_config &c, CkptLayout &l) {
  if (c.dim <= 0 || c.hidden_dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
      c.vocab_size == 0 || c.seq_len <= 0 || c.dim % c.n_heads || c.n_heads % c.n_kv_heads)
    return set_error(SIMP_RT_EINVAL, "checkpoint: inconsistent config header");
  const int64_t dim = c.dim, hid = c.hidden_dim, L = c.n_layers, V = std::abs((int64_t)c.vocab_size);
  const int64_t hs = dim / c.n_heads, kvd = dim * c.n_kv_heads / c.n_heads;
  l.shared = c.vocab_size > 0;
  l.emb = V * dim;
  l.rms_att = L * dim;
  l.wq = L * dim * dim;
  l.wk = L * kvd * dim;
  l.wv = L * kvd * dim;
  l.wo = L * dim * dim;
  l.rms_ffn = L * dim;
  l.w1 = L * hid * dim;
  l.w2 = L * dim * hid;
  l.w3 = L * hid * dim;
  l.rms_final = dim;
  l.freq = l.shared ? 0 : c.seq_len * hs;  // legacy freq_cis_real + _imag, skipped
  l.wcls = l.shared ? 0 : V * dim;
  return SIMP_RT_OK;
}

// Packed W4 model files.  A 64-byte header (8-byte magic, the llama2.c
// config as 7 int32, the group size, zero padding), then the sections in a
// fixed order, each padded to a multiple of 256 bytes so that every array is
// 16-byte aligned when the file is read into one device allocation.
constexpr size_t kHdr = 64, kAlign = 256;
inline size_t pad_to(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

struct W4Header {
  char magic[8];
  simp_rt_ckpt_config cfg;
  int32_t group_size;
};

int write_padded(FILE *f, const void *host, size_t bytes) {
  static const char zeros[kAlign] = {};
  if (bytes && fwrite(host, 1, bytes, f) != bytes) return -1;
  const size_t pad = pad_to(bytes) - bytes;
  if (pad && fwrite(zeros, 1, pad, f) != pad) return -1;
  return 0;
}

int write_device_padded(FILE *f, const void *dev, size_t bytes, const char *what) {
  std::vector<char> h(bytes);
  if (bytes && hipMemcpy(h.data(), dev, bytes, hipMemcpyDeviceToHost) != hipSuccess)
    return set_error(SIMP_RT_EHIP, "%s: device read-back", what);
  if (write_padded(f, h.data(), bytes)) return set_error(SIMP_RT_EINVAL, "%s: write failed", what);
  return SIMP_RT_OK;
}

// Header + whole body of a packed model file into one device allocation.
int read_w4_file(const char *path, const char *magic, W4Header &hdr, char **body, size_t &body_bytes,
                 const char *what) {
  FileCloser fc{fopen(path, "rb")};
  if (!fc.f) return set_error(SIMP_RT_EINVAL, "%s: cannot open %s", what, path);
  char raw[kHdr];
  if (fread(raw, 1, kHdr, fc.f) != kHdr) return set_error(SIMP_RT_EINVAL, "%s: %s has no header", what, path);
  memcpy(&hdr, raw, sizeof(hdr));
  if (memcmp(hdr.magic, magic, 8)) return set_error(SIMP_RT_EINVAL, "%s: %s is not a %.8s file", what, path, magic);
  if (fseek(fc.f, 0, SEEK_END)) return set_error(SIMP_RT_EINVAL, "%s: cannot size %s", what, path);
  const long end = ftell(fc.f);
  if (end < (long)kHdr || fseek(fc.f, (long)kHdr, SEEK_SET))
    return set_error(SIMP_RT_EINVAL, "%s: cannot size %s", what, path);
  body_bytes = (size_t)end - kHdr;
  if (hipMalloc((void **)body, std::max<size_t>(body_bytes, 16)) != hipSuccess)
    return set_error(SIMP_RT_ENOMEM, "%s: %zu bytes of device memory", what, body_bytes);
  int rc = read_to_device(fc.f, *body, body_bytes, cur_stream(), what);
  if (rc) {
    (void)hipFree(*body);
    *body = nullptr;
  }
  return rc;
}

struct TokenizerImpl {
  std::vector<std::string> vocab;
  std::vector<float> scores;
  int32_t max_token_length = 0;
};

struct SamplerImpl {
  std::mt19937 rng;
  std::vector<float> p;
};

}  // namespace
}  // namespace simp

using namespace simp;

struct simp_rt_tokenizer {
  TokenizerImpl t;
};
struct simp_rt_sampler {
  SamplerImpl s;
};

extern "C" {

int32_t simp_rt_ckpt_read_config(const char *path, simp_rt_ckpt_config *cfg) {
  if (!path || !cfg) return set_error(SIMP_RT_EINVAL, "ckpt_read_config: null argument");
  FileCloser fc{fopen(path, "rb")};
  if (!fc.f) return set_error(SIMP_RT_EINVAL, "ckpt_read_config: cannot open %s", path);
  if (fread(cfg, sizeof(*cfg), 1, fc.f) != 1)
    return set_error(SIMP_RT_EINVAL, "ckpt_read_config: %s is shorter than its header", path);
  CkptLayout l;
  return ckpt_layout(*cfg, l);
}

int32_t simp_rt_ckpt_load_f32(const char *path, simp_rt_ckpt_config *cfg, simp_rt_llama_weights *w,
                              void **blob) {
  if (!path || !cfg || !w || !blob) return set_error(SIMP_RT_EINVAL, "ckpt_load_f32: null argument");
  *blob = nullptr;
  int rc;
  if ((rc = ensure_device())) return rc;
  FileCloser fc{fopen(path, "rb")};
  if (!fc.f) return set_error(SIMP_RT_EINVAL, "ckpt_load_f32: cannot open %s", path);
  if (fread(cfg, sizeof(*cfg), 1, fc.f) != 1)
    return set_error(SIMP_RT_EINVAL, "ckpt_load_f32: %s is shorter than its header", path);
  CkptLayout l;
  if ((rc = ckpt_layout(*cfg, l))) return rc;
  const size_t bytes = sizeof(float) * (size_t)l.total();
  float *d = nullptr;
  if (hipMalloc((void **)&d, bytes) != hipSuccess)
    return set_error(SIMP_RT_ENOMEM, "ckpt_load_f32: %zu bytes of device memory", bytes);
  if ((rc = read_to_device(fc.f, d, bytes, cur_stream(), "ckpt_load_f32"))) {
    (void)hipFree(d);
    return rc;
  }
  memset(w, 0, sizeof(*w));
  const float *p = d;
  auto take = [&](int64_t n) {
    const float *r = p;
    p += n;
    return r;
  };
  w->token_embedding = take(l.emb);
  w->rms_att = take(l.rms_att);
  w->wq = take(l.wq);
  w->wk = take(l.wk);
  w->wv = take(l.wv);
  w->wo = take(l.wo);
  w->rms_ffn = take(l.rms_ffn);
  w->w1 = take(l.w1);
  w->w2 = take(l.w2);
  w->w3 = take(l.w3);
  w->rms_final = take(l.rms_final);
  take(l.freq);
  w->wcls = l.shared ? w->token_embedding : take(l.wcls);
  *blob = d;
  return SIMP_RT_OK;
}

int32_t simp_rt_tokenizer_load(const char *path, int32_t vocab_size, simp_rt_tokenizer **tok) {
  if (!path || !tok || vocab_size <= 0) return set_error(SIMP_RT_EINVAL, "tokenizer_load: bad argument");
  *tok = nullptr;
  FileCloser fc{fopen(path, "rb")};
  if (!fc.f) return set_error(SIMP_RT_EINVAL, "tokenizer_load: cannot open %s", path);
  auto *t = new simp_rt_tokenizer();
  if (fread(&t->t.max_token_length, 4, 1, fc.f) != 1) {
    delete t;
    return set_error(SIMP_RT_EINVAL, "tokenizer_load: %s is empty", path);
  }
  t->t.vocab.reserve(vocab_size);
  t->t.scores.reserve(vocab_size);
  for (int32_t i = 0; i < vocab_size; i++) {
    float score;
    int32_t len;
    if (fread(&score, 4, 1, fc.f) != 1 || fread(&len, 4, 1, fc.f) != 1 || len < 0) {
      delete t;
      return set_error(SIMP_RT_EINVAL, "tokenizer_load: %s ends at token %d of %d", path, i, vocab_size);
    }
    std::string s((size_t)len, '\0');
    if (len && fread(&s[0], 1, (size_t)len, fc.f) != (size_t)len) {
      delete t;
      return set_error(SIMP_RT_EINVAL, "tokenizer_load: %s ends inside token %d", path, i);
    }
    t->t.scores.push_back(score);
    t->t.vocab.push_back(std::move(s));
  }
  *tok = t;
  return SIMP_RT_OK;
}

const char *simp_rt_tokenizer_decode(const simp_rt_tokenizer *tok, int32_t token, int32_t *len) {
  static const char kUnknown[] = "?";
  if (!tok || token < 0 || token >= (int32_t)tok->t.vocab.size()) {
    if (len) *len = 1;
    return kUnknown;
  }
  const std::string &s = tok->t.vocab[token];
  if (len) *len = (int32_t)s.size();
  return s.data();
}

float simp_rt_tokenizer_score(const simp_rt_tokenizer *tok, int32_t token) {
  if (!tok || token < 0 || token >= (int32_t)tok->t.scores.size()) return NAN;
  return tok->t.scores[token];
}

int32_t simp_rt_tokenizer_max_token_length(const simp_rt_tokenizer *tok) {
  return tok ? tok->t.max_token_length : SIMP_RT_EINVAL;
}

int32_t simp_rt_tokenizer_free(simp_rt_tokenizer *tok) {
  delete tok;
  return SIMP_RT_OK;
}

int32_t simp_rt_sampler_create(uint32_t seed, simp_rt_sampler **s) {
  if (!s) return set_error(SIMP_RT_EINVAL, "sampler_create: null argument");
  *s = new simp_rt_sampler();
  (*s)->s.rng.seed(seed);
  return SIMP_RT_OK;
}

int32_t simp_rt_sampler_sample(simp_rt_sampler *s, const float *logits, int32_t n, float temperature) {
  if (!s || !logits || n <= 0) return set_error(SIMP_RT_EINVAL, "sampler_sample: bad argument");
  if (temperature == 0.0f) {
    int best = 0;
    float bv = logits[0];
    for (int i = 1; i < n; i++)
      if (logits[i] > bv) {
        bv = logits[i];
        best = i;
      }
    return best;
  }
  std::vector<float> &p = s->s.p;
  p.assign(logits, logits + n);
  for (int i = 0; i < n; i++) p[i] /= temperature;
  const float mx = *std::max_element(p.begin(), p.end());
  float sum = 0.0f;
  for (int i = 0; i < n; i++) {
    p[i] = expf(p[i] - mx);
    sum += p[i];
  }
  for (int i = 0; i < n; i++) p[i] /= sum;
  std::uniform_real_distribution<float> dist(0.0f, 1.0f);
  const float r = dist(s->s.rng);
  float cdf = 0.0f;
  for (int i = 0; i < n; i++) {
    cdf += p[i];
    if (r < cdf) return i;
  }
  return n - 1;
}

int32_t simp_rt_sampler_free(simp_rt_sampler *s) {
  delete s;
  return SIMP_RT_OK;
}

int32_t simp_rt_quantize_w4u(const float *w, int64_t n, int32_t group_size, uint8_t *q, float *scales,
                             float *zeros) {
  if (!w || !q || !scales || !zeros || n <= 0 || group_size <= 0 || group_size % 2)
    return set_error(SIMP_RT_EINVAL, "quantize_w4u: bad argument (group_size must be even)");
  int rc;
  if ((rc = ensure_device())) return rc;
  const int64_t ngroups = (n + group_size - 1) / group_size;
  hipLaunchKernelGGL(quant_w4u_k, dim3((unsigned)cdiv(ngroups, 4)), dim3(256), 0, cur_stream(), w, n,
                     (int)group_size, q, scales, zeros);
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}

int32_t simp_rt_quantize_w4s(const float *w, int64_t rows, int64_t cols, int32_t group_size, uint8_t *q,
                             float *scales) {
  if (!w || !q || !scales || rows <= 0 || cols <= 0 || group_size <= 0 || group_size % 2 ||
      cols % group_size)
    return set_error(SIMP_RT_EINVAL, "quantize_w4s: bad argument (cols must be a multiple of an even group_size)");
  int rc;
  if ((rc = ensure_device())) return rc;
  const int64_t t = rows * (cols / group_size);
  hipLaunchKernelGGL(quant_w4s_k, dim3((unsigned)cdiv(t, 4)), dim3(256), 0, cur_stream(), w, rows, cols,
                     (int)group_size, q, scales);
  SIMP_HIP(hipGetLastError());
  return SIMP_RT_OK;
}


int32_t simp_rt_w4s_file_write(const char *ckpt_path, const char *out_path, int32_t group_size) {
  static const char *kWhat = "w4s_file_write";
  if (!ckpt_path || !out_path || group_size <= 0 || group_size % 32)
    return set_error(SIMP_RT_EINVAL, "%s: bad argument (group_size: a multiple of 32)", kWhat);
  simp_rt_ckpt_config cfg;
  simp_rt_llama_weights w;
  void *blob = nullptr;
  int rc;
  if ((rc = simp_rt_ckpt_load_f32(ckpt_path, &cfg, &w, &blob))) return rc;
  const int64_t dim = cfg.dim, hid = cfg.hidden_dim, L = cfg.n_layers, V = std::abs((int64_t)cfg.vocab_size);
  const int64_t kvd = dim * cfg.n_kv_heads / cfg.n_heads;
  struct Mat { const float *src; int64_t rows, cols; };
  const Mat mats[8] = {{w.wq, L * dim, dim},  {w.wk, L * kvd, dim}, {w.wv, L * kvd, dim},
                       {w.wo, L * dim, dim},  {w.w1, L * hid, dim}, {w.w2, L * dim, hid},
                       {w.w3, L * hid, dim},  {w.wcls, V, dim}};
  for (const Mat &m : mats)
    if (m.cols % group_size) {
      (void)hipFree(blob);
      return set_error(SIMP_RT_EINVAL, "%s: dim and hidden_dim must be multiples of group_size %d", kWhat,
                       group_size);
    }
  FileCloser fc{fopen(out_path, "wb")};
  if (!fc.f) {
    (void)hipFree(blob);
    return set_error(SIMP_RT_EINVAL, "%s: cannot create %s", kWhat, out_path);
  }
  char raw[kHdr] = {};
  W4Header hdr;
  memcpy(hdr.magic, "SIMPW4S1", 8);
  hdr.cfg = cfg;
  hdr.cfg.vocab_size = (int32_t)V;
  hdr.group_size = group_size;
  memcpy(raw, &hdr, sizeof(hdr));
  if (fwrite(raw, 1, kHdr, fc.f) != kHdr) rc = set_error(SIMP_RT_EINVAL, "%s: write failed", kWhat);
  const struct { const float *p; int64_t n; } f32s[4] = {
      {w.token_embedding, V * dim}, {w.rms_att, L * dim}, {w.rms_ffn, L * dim}, {w.rms_final, dim}};
  for (const auto &a : f32s)
    if (!rc) rc = write_device_padded(fc.f, a.p, sizeof(float) * (size_t)a.n, kWhat);
  uint8_t *q = nullptr;
  float *sc = nullptr;
  for (const Mat &m : mats) {
    if (rc) break;
    const size_t qb = (size_t)(m.rows * m.cols / 2), sb = sizeof(float) * (size_t)(m.rows * m.cols / group_size);
    if (hipMalloc((void **)&q, qb) != hipSuccess || hipMalloc((void **)&sc, sb) != hipSuccess) {
      rc = set_error(SIMP_RT_ENOMEM, "%s: quantization buffers", kWhat);
      break;
    }
    if (!(rc = simp_rt_quantize_w4s(m.src, m.rows, m.cols, group_size, q, sc)) &&
        !(rc = write_device_padded(fc.f, q, qb, kWhat)))
      rc = write_device_padded(fc.f, sc, sb, kWhat);
    (void)hipFree(q);
    (void)hipFree(sc);
    q = nullptr;
    sc = nullptr;
  }
  (void)hipFree(blob);
  return rc;
}

int32_t simp_rt_w4s_file_load(const char *path, simp_rt_llama_config *cfg, simp_rt_llama_weights *w,
                              void **blob) {
  static const char *kWhat = "w4s_file_load";
  if (!path || !cfg || !w || !blob) return set_error(SIMP_RT_EINVAL, "%s: null argument", kWhat);
  *blob = nullptr;
  int rc;
  if ((rc = ensure_device())) return rc;
  W4Header hdr;
  char *body = nullptr;
  size_t bytes = 0;
  if ((rc = read_w4_file(path, "SIMPW4S1", hdr, &body, bytes, kWhat))) return rc;
  const simp_rt_ckpt_config &c = hdr.cfg;
  CkptLayout l;
  const int gs = hdr.group_size;
  if ((rc = ckpt_layout(c, l)) || gs <= 0 || gs % 32 || c.vocab_size <= 0) {
    (void)hipFree(body);
    return rc ? rc : set_error(SIMP_RT_EINVAL, "%s: bad header in %s", kWhat, path);
  }
  const int64_t dim = c.dim, hid = c.hidden_dim, L = c.n_layers, V = c.vocab_size;
  const int64_t kvd = dim * c.n_kv_heads / c.n_heads;
  size_t off = 0;
  bool short_file = false;
  auto take = [&](size_t n) {
    const char *p = body + off;
    off += pad_to(n);
    if (off > bytes) short_file = true;
    return p;
  };
  memset(w, 0, sizeof(*w));
  w->token_embedding = (const float *)take(4 * (size_t)(V * dim));
  w->rms_att = (const float *)take(4 * (size_t)(L * dim));
  w->rms_ffn = (const float *)take(4 * (size_t)(L * dim));
  w->rms_final = (const float *)take(4 * (size_t)dim);
  const int64_t rc_[8][2] = {{L * dim, dim}, {L * kvd, dim}, {L * kvd, dim}, {L * dim, dim},
                             {L * hid, dim}, {L * dim, hid}, {L * hid, dim}, {V, dim}};
  const uint8_t **qs[8] = {&w->q_wq, &w->q_wk, &w->q_wv, &w->q_wo, &w->q_w1, &w->q_w2, &w->q_w3, &w->q_wcls};
  const float **ss[8] = {&w->s_wq, &w->s_wk, &w->s_wv, &w->s_wo, &w->s_w1, &w->s_w2, &w->s_w3, &w->s_wcls};
  for (int i = 0; i < 8; i++) {
    *qs[i] = (const uint8_t *)take((size_t)(rc_[i][0] * rc_[i][1] / 2));
    *ss[i] = (const float *)take(4 * (size_t)(rc_[i][0] * rc_[i][1] / gs));
  }
  if (short_file) {
    (void)hipFree(body);
    memset(w, 0, sizeof(*w));
    return set_error(SIMP_RT_EINVAL, "%s: %s is shorter than its header says", kWhat, path);
  }
  memset(cfg, 0, sizeof(*cfg));
  cfg->dim = dim;
  cfg->hidden_dim = hid;
  cfg->n_layers = L;
  cfg->n_heads = c.n_heads;
  cfg->n_kv_heads = c.n_kv_heads;
  cfg->vocab_size = V;
  cfg->seq_len = c.seq_len;
  cfg->eps = 1e-5f;
  cfg->rope_theta = 10000.f;
  cfg->weight_format = SIMP_RT_W_W4S;
  cfg->group_size = gs;
  *blob = body;
  return SIMP_RT_OK;
}

int32_t simp_rt_w4u_file_write(const char *ckpt_path, const char *out_path, int32_t group_size) {
  static const char *kWhat = "w4u_file_write";
  if (!ckpt_path || !out_path || group_size <= 0 || group_size % 2)
    return set_error(SIMP_RT_EINVAL, "%s: bad argument (group_size must be even)", kWhat);
  simp_rt_ckpt_config cfg;
  simp_rt_llama_weights w;
  void *blob = nullptr;
  int rc;
  if ((rc = simp_rt_ckpt_load_f32(ckpt_path, &cfg, &w, &blob))) return rc;
  const int64_t dim = cfg.dim, hid = cfg.hidden_dim, L = cfg.n_layers, V = std::abs((int64_t)cfg.vocab_size);
  const int64_t kvd = dim * cfg.n_kv_heads / cfg.n_heads;
  // the reference quantizes each tensor type (all layers) with quantize_w4 and
  // appends it: qweights byte offsets and scale/zero indices restart per tensor
  const struct { const float *src; int64_t n; } ts[7] = {{w.wq, L * dim * dim}, {w.wk, L * kvd * dim},
                                                         {w.wv, L * kvd * dim}, {w.wo, L * dim * dim},
                                                         {w.w1, L * hid * dim}, {w.w2, L * dim * hid},
                                                         {w.w3, L * hid * dim}};
  int64_t qbytes = 0, ngroups = 0, offs[7], goffs[7];
  for (int i = 0; i < 7; i++) {
    offs[i] = 2 * qbytes;  // element offset of the tensor in qweights
    goffs[i] = ngroups;
    qbytes += (ts[i].n + 1) / 2;
    ngroups += (ts[i].n + group_size - 1) / group_size;
  }
  uint8_t *q = nullptr;
  float *sc = nullptr, *zr = nullptr;
  if (hipMalloc((void **)&q, qbytes) != hipSuccess || hipMalloc((void **)&sc, 4 * ngroups) != hipSuccess ||
      hipMalloc((void **)&zr, 4 * ngroups) != hipSuccess)
    rc = set_error(SIMP_RT_ENOMEM, "%s: quantization buffers", kWhat);
  for (int i = 0; i < 7 && !rc; i++)
    rc = simp_rt_quantize_w4u(ts[i].src, ts[i].n, group_size, q + offs[i] / 2, sc + goffs[i], zr + goffs[i]);
  FileCloser fc{rc ? nullptr : fopen(out_path, "wb")};
  if (!rc && !fc.f) rc = set_error(SIMP_RT_EINVAL, "%s: cannot create %s", kWhat, out_path);
  if (!rc) {
    char raw[kHdr] = {};
    W4Header hdr;
    memcpy(hdr.magic, "SIMPW4U1", 8);
    hdr.cfg = cfg;
    hdr.cfg.vocab_size = (int32_t)V;
    hdr.group_size = group_size;
    memcpy(raw, &hdr, sizeof(hdr));
    if (fwrite(raw, 1, kHdr, fc.f) != kHdr || write_padded(fc.f, offs, sizeof(offs)))
      rc = set_error(SIMP_RT_EINVAL, "%s: write failed", kWhat);
    const struct { const void *p; size_t n; } secs[8] = {
        {w.token_embedding, 4 * (size_t)(V * dim)}, {w.rms_att, 4 * (size_t)(L * dim)},
        {w.rms_ffn, 4 * (size_t)(L * dim)},         {w.rms_final, 4 * (size_t)dim},
        {w.wcls, 4 * (size_t)(V * dim)},            {q, (size_t)qbytes},
        {sc, 4 * (size_t)ngroups},                  {zr, 4 * (size_t)ngroups}};
    for (const auto &sct : secs)
      if (!rc) rc = write_device_padded(fc.f, sct.p, sct.n, kWhat);
  }
  if (q) (void)hipFree(q);
  if (sc) (void)hipFree(sc);
  if (zr) (void)hipFree(zr);
  (void)hipFree(blob);
  return rc;
}

int32_t simp_rt_w4u_file_load(const char *path, simp_rt_w4u_model *m, void **blob) {
  static const char *kWhat = "w4u_file_load";
  if (!path || !m || !blob) return set_error(SIMP_RT_EINVAL, "%s: null argument", kWhat);
  *blob = nullptr;
  int rc;
  if ((rc = ensure_device())) return rc;
  W4Header hdr;
  char *body = nullptr;
  size_t bytes = 0;
  if ((rc = read_w4_file(path, "SIMPW4U1", hdr, &body, bytes, kWhat))) return rc;
  const simp_rt_ckpt_config &c = hdr.cfg;
  CkptLayout l;
  if ((rc = ckpt_layout(c, l)) || hdr.group_size <= 0 || hdr.group_size % 2 || c.vocab_size <= 0) {
    (void)hipFree(body);
    return rc ? rc : set_error(SIMP_RT_EINVAL, "%s: bad header in %s", kWhat, path);
  }
  const int64_t dim = c.dim, hid = c.hidden_dim, L = c.n_layers, V = c.vocab_size;
  const int64_t kvd = dim * c.n_kv_heads / c.n_heads;
  const int64_t ns[7] = {L * dim * dim, L * kvd * dim, L * kvd * dim, L * dim * dim,
                         L * hid * dim, L * dim * hid, L * hid * dim};
  int64_t qbytes = 0, ngroups = 0;
  for (int i = 0; i < 7; i++) {
    qbytes += (ns[i] + 1) / 2;
    ngroups += (ns[i] + hdr.group_size - 1) / hdr.group_size;
  }
  size_t off = 0;
  bool short_file = false;
  auto take = [&](size_t n) {
    const char *p = body + off;
    off += pad_to(n);
    if (off > bytes) short_file = true;
    return p;
  };
  memset(m, 0, sizeof(*m));
  const char *offs_dev = take(sizeof(m->offsets));
  m->token_embedding = (const float *)take(4 * (size_t)(V * dim));
  m->rms_att = (const float *)take(4 * (size_t)(L * dim));
  m->rms_ffn = (const float *)take(4 * (size_t)(L * dim));
  m->rms_final = (const float *)take(4 * (size_t)dim);
  m->wcls = (const float *)take(4 * (size_t)(V * dim));
  m->qweights = (const int8_t *)take((size_t)qbytes);
  m->scales = (const float *)take(4 * (size_t)ngroups);
  m->zeros = (const float *)take(4 * (size_t)ngroups);
  if (short_file || hipMemcpy(m->offsets, offs_dev, sizeof(m->offsets), hipMemcpyDeviceToHost) != hipSuccess) {
    (void)hipFree(body);
    memset(m, 0, sizeof(*m));
    return set_error(SIMP_RT_EINVAL, "%s: %s is shorter than its header says", kWhat, path);
  }
  m->dim = dim;
  m->hidden_dim = hid;
  m->n_layers = L;
  m->n_heads = c.n_heads;
  m->n_kv_heads = c.n_kv_heads;
  m->vocab_size = V;
  m->seq_len = c.seq_len;
  m->group_size = hdr.group_size;
  m->qweights_bytes = qbytes;
  m->n_groups = ngroups;
  *blob = body;
  return SIMP_RT_OK;
}

}  // extern "C"
