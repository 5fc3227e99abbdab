// CPU restatement of MuNet's CPU-backend arithmetic, used ONLY as the parity
// checker for the HIP backend (test infrastructure, never linked into the
// product library). Every function names the reference code it restates.
//
// Semantics restated (reference paths, /root/reference):
//   * dtype codecs ............ src/types.hpp:239-317 (fp16 round-half-away,
//                               bf16 RNE without NaN special case)
//   * scalar read/write ....... src/types.hpp:326-395 (double -> float -> codec)
//   * fp32 matmul ............. src/backend/cpu_backend.hpp:334-374 (float sum,
//                               k order) and ops/common.hpp:276-289 (batched)
//   * fp16 matmul ............. src/core/ops/matmul.cpp:25-84,132-228 (convert
//                               to fp32, fp32 loop, round-half-away back)
//   * bf16 matmul ............. src/core/ops/common.hpp:128-256 (double sum)
//   * binary broadcast ........ src/backend/cpu_backend.hpp:238-332 (fp32),
//                               src/core/ops/common.hpp:46-85 (fp16/bf16)
//   * relu/sigmoid ............ cpu_backend.hpp:493-531, activations.cpp:26-64
//   * softmax ................. cpu_backend.hpp:587-611, activations.cpp:189-254
//   * layer_norm .............. src/core/ops/normalization.cpp:125-224 (double)
//   * masked_fill ............. src/core/ops/elementwise.cpp:8-53
//   * MHA core ................ src/nn/attention.hpp:34-104 (K-reinterpretation,
//                               dense block-diagonal mask, -1e9 fill)
//   * embedding gather ........ src/nn/linear.hpp:92-128
//   * conv2d / pool / upsample  cpu_backend.hpp:768-902, ops/conv2d.cpp:51-72,
//                               ops/pooling.cpp:8-93
//   * concat .................. cpu_backend.hpp:416-452 (copy)
// Work is split across threads only over independent output elements, so the
// per-element operation order (and hence every bit) matches the reference.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>
#include <algorithm>
#include <functional>

namespace {

enum DType { F32 = 0, F16 = 1, BF16 = 2, I32 = 3 };

thread_local std::string g_err;

size_t dsize(int dt) { return (dt == F16 || dt == BF16) ? 2 : 4; }

// ---- codecs (restating src/types.hpp:239-317) ------------------------------
uint16_t enc_f16(float value) {
  uint32_t bits;
  std::memcpy(&bits, &value, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t raw_exp = (bits >> 23) & 0xffu;
  uint32_t man = bits & 0x7fffffu;
  int e = int(raw_exp) - 127 + 15;
  if (raw_exp == 0xffu) return uint16_t(sign | (man ? 0x7e00u : 0x7c00u));
  if (e <= 0) {
    if (e < -10) return uint16_t(sign);
    man |= 0x800000u;
    uint32_t sh = man >> uint32_t(1 - e);
    return uint16_t(sign | ((sh + 0x1000u) >> 13));
  }
  if (e >= 31) return uint16_t(sign | 0x7c00u);
  uint32_t rm = (man + 0x1000u) >> 13;
  if (rm == 0x400u) {
    ++e;
    if (e >= 31) return uint16_t(sign | 0x7c00u);
    return uint16_t(sign | (uint32_t(e) << 10));
  }
  return uint16_t(sign | (uint32_t(e) << 10) | (rm & 0x3ffu));
}

float dec_f16(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      // subnormal: value = m * 2^-24, renormalise
      uint32_t mm = m;
      int shift = 0;
      while ((mm & 0x400u) == 0) { mm <<= 1; ++shift; }
      bits = sign | (uint32_t(127 - 15 - shift + 1) << 23) | ((mm & 0x3ffu) << 13);
    }
  } else if (e == 0x1fu) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

uint16_t enc_bf16(float value) {
  uint32_t bits;
  std::memcpy(&bits, &value, 4);
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return uint16_t(bits >> 16);
}

float dec_bf16(uint16_t b) {
  uint32_t bits = uint32_t(b) << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

inline double rd(const void *p, int dt, size_t i) {
  switch (dt) {
  case F32: return double(static_cast<const float *>(p)[i]);
  case F16: return double(dec_f16(static_cast<const uint16_t *>(p)[i]));
  case BF16: return double(dec_bf16(static_cast<const uint16_t *>(p)[i]));
  case I32: return double(static_cast<const int32_t *>(p)[i]);
  }
  throw std::runtime_error("bad dtype");
}

inline void wr(void *p, int dt, size_t i, double v) {
  switch (dt) {
  case F32: static_cast<float *>(p)[i] = float(v); return;
  case F16: static_cast<uint16_t *>(p)[i] = enc_f16(float(v)); return;
  case BF16: static_cast<uint16_t *>(p)[i] = enc_bf16(float(v)); return;
  case I32: static_cast<int32_t *>(p)[i] = int32_t(v); return;
  }
  throw std::runtime_error("bad dtype");
}

// Which threading the reference gives a loop (src/backend/cpu_backend.hpp:
// 101-127): BACKEND loops run in CPUBackend::parallel_for (inline below 1024
// iterations, otherwise blocks over hardware_concurrency() threads); SERIAL
// loops are the typed fallbacks and host-side ops (ops/common.hpp:46-289,
// ops/normalization.cpp:125-224, ops/elementwise.cpp:8-53), which never split.
enum Path { BACKEND = 0, SERIAL = 1 };

// 0 = parity mode: every loop over independent outputs is split over all
//     hardware threads once it has 64 iterations (fast checking);
// 1 = reference mode: the reference's own split per Path (the timed CPU
//     baseline).  Either way each output element's operation order, and so
//     every bit, is the reference's.
int g_threading = 0;

void par_for(size_t n, const std::function<void(size_t, size_t)> &fn, Path path = BACKEND) {
  unsigned nt = std::max(1u, std::thread::hardware_concurrency());
  if (g_threading == 1) {
    if (path == SERIAL || n < 1024 || nt == 1) { fn(0, n); return; }
  } else if (n < 64 || nt == 1) {
    fn(0, n);
    return;
  }
  nt = unsigned(std::min<size_t>(nt, n));
  std::vector<std::thread> th;
  size_t blk = (n + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    size_t s = t * blk, e = std::min(n, s + blk);
    if (s >= e) break;
    th.emplace_back([&, s, e] { fn(s, e); });
  }
  for (auto &x : th) x.join();
}

std::vector<float> to_f32(const void *p, int dt, size_t n) {
  std::vector<float> out(n);
  for (size_t i = 0; i < n; ++i) out[i] = float(rd(p, dt, i));
  return out;
}

// ---- matmul core (one [M,K]x[K,N] product per batch slice) -----------------
// fp32 / fp16: float accumulation in k order (cpu_backend.hpp:350-373,
// common.hpp:276-289); fp16 rounds the float result with round-half-away.
// bf16: double accumulation, then double->float->bf16 (common.hpp:128-165).

// Parity-mode product over rows [r0, r1) of one slice: the row of A and the
// transposed B (bt, [N, K]) are k-contiguous exact copies of the operands, and
// eight output columns run side by side, each its own sum in k order -- the
// operations of the reference's i-n-k loop, only laid out for the cache.
template <typename T, typename Store>
void product_rows(const T *a, const T *bt, int M, int K, int N, bool transA,
                  size_t r0, size_t r1, Store store) {
  std::vector<T> arow(K);
  for (size_t m = r0; m < r1; ++m) {
    for (int k = 0; k < K; ++k) arow[k] = transA ? a[size_t(k) * M + m] : a[m * K + k];
    int n = 0;
    for (; n + 8 <= N; n += 8) {
      const T *b0 = bt + size_t(n) * K, *b1 = b0 + K, *b2 = b1 + K, *b3 = b2 + K;
      const T *b4 = b3 + K, *b5 = b4 + K, *b6 = b5 + K, *b7 = b6 + K;
      T s0 = 0, s1 = 0, s2 = 0, s3 = 0, s4 = 0, s5 = 0, s6 = 0, s7 = 0;
      for (int k = 0; k < K; ++k) {
        const T x = arow[k];
        s0 += x * b0[k];
        s1 += x * b1[k];
        s2 += x * b2[k];
        s3 += x * b3[k];
        s4 += x * b4[k];
        s5 += x * b5[k];
        s6 += x * b6[k];
        s7 += x * b7[k];
      }
      store(m, n, s0);
      store(m, n + 1, s1);
      store(m, n + 2, s2);
      store(m, n + 3, s3);
      store(m, n + 4, s4);
      store(m, n + 5, s5);
      store(m, n + 6, s6);
      store(m, n + 7, s7);
    }
    for (; n < N; ++n) {
      const T *b0 = bt + size_t(n) * K;
      T s0 = 0;
      for (int k = 0; k < K; ++k) s0 += arow[k] * b0[k];
      store(m, n, s0);
    }
  }
}

// Parity mode: decode both operands once (exact) into T, B transposed.
template <typename T>
void matmul_parity(int dt, const void *A, const void *B, void *C, int batch, int M,
                   int K, int N, bool b_batched, bool transA, bool transB) {
  const size_t sa = size_t(M) * K, sb = size_t(K) * N, sc = size_t(M) * N;
  const int nb = b_batched ? batch : 1;
  std::vector<T> ad(sa * batch), bt(sb * nb);
  par_for(ad.size(), [&](size_t s, size_t e) {
    for (size_t i = s; i < e; ++i) ad[i] = T(rd(A, dt, i));
  });
  par_for(size_t(nb) * N, [&](size_t s, size_t e) {
    for (size_t r = s; r < e; ++r) {
      size_t bi = r / N, n = r % N;
      for (int k = 0; k < K; ++k)
        bt[bi * sb + n * K + k] =
            T(rd(B, dt, bi * sb + (transB ? n * K + k : size_t(k) * N + n)));
    }
  });
  for (int bi = 0; bi < batch; ++bi) {
    const T *a = ad.data() + bi * sa, *b = bt.data() + (b_batched ? bi * sb : 0);
    par_for(size_t(M), [&](size_t s, size_t e) {
      product_rows<T>(a, b, M, K, N, transA, s, e, [&](size_t m, int n, T v) {
        const size_t o = bi * sc + m * N + n;
        if (dt == F32)
          static_cast<float *>(C)[o] = float(v);
        else if (dt == F16)
          static_cast<uint16_t *>(C)[o] = enc_f16(float(v));
        else
          wr(C, dt, o, double(v));
      });
    });
  }
}

void matmul_slices(int dt, const void *A, const void *B, void *C, int batch,
                   int M, int K, int N, bool b_batched, bool transA,
                   bool transB) {
  if (g_threading == 0) {
    if (dt == BF16)
      matmul_parity<double>(dt, A, B, C, batch, M, K, N, b_batched, transA, transB);
    else
      matmul_parity<float>(dt, A, B, C, batch, M, K, N, b_batched, transA, transB);
    return;
  }
  // Reference mode: the reference's loops as they run.
  const size_t sa = size_t(M) * K, sb = b_batched ? size_t(K) * N : 0,
               sc = size_t(M) * N;
  if (dt == F32 || dt == F16) {
    std::vector<float> af, bf;
    const float *ap, *bp;
    if (dt == F16) {
      af = to_f32(A, dt, sa * batch);
      bf = to_f32(B, dt, b_batched ? sb * batch : size_t(K) * N);
      ap = af.data();
      bp = bf.data();
    } else {
      ap = static_cast<const float *>(A);
      bp = static_cast<const float *>(B);
    }
    par_for(size_t(batch) * M, [&](size_t s, size_t e) {
      for (size_t r = s; r < e; ++r) {
        size_t bi = r / M, m = r % M;
        const float *a = ap + bi * sa, *b = bp + bi * sb;
        for (int n = 0; n < N; ++n) {
          float sum = 0.0f;
          for (int k = 0; k < K; ++k) {
            float av = transA ? a[size_t(k) * M + m] : a[m * K + k];
            float bv = transB ? b[size_t(n) * K + k] : b[size_t(k) * N + n];
            sum += av * bv;
          }
          if (dt == F32)
            static_cast<float *>(C)[bi * sc + m * N + n] = sum;
          else
            static_cast<uint16_t *>(C)[bi * sc + m * N + n] = enc_f16(sum);
        }
      }
    }, batch > 1 ? SERIAL : BACKEND);
    return;
  }
  // bf16: the serial scalar fallback exactly as it runs (ops/common.hpp:
  // 146-160), each operand read and decoded per product.
  for (int bi = 0; bi < batch; ++bi)
    for (int m = 0; m < M; ++m)
      for (int n = 0; n < N; ++n) {
        double sum = 0.0;
        for (int k = 0; k < K; ++k) {
          size_t ai = bi * sa + (transA ? size_t(k) * M + m : size_t(m) * K + k);
          size_t bidx = bi * sb + (transB ? size_t(n) * K + k : size_t(k) * N + n);
          sum += rd(A, dt, ai) * rd(B, dt, bidx);
        }
        wr(C, dt, bi * sc + size_t(m) * N + n, sum);
      }
}

enum BinOp { ADD = 0, SUB = 1, MUL = 2, DIV = 3 };

template <typename T> T binop(int op, T a, T b) {
  switch (op) {
  case ADD: return a + b;
  case SUB: return a - b;
  case MUL: return a * b;
  default: return a / b;
  }
}

// compute_broadcast (types.hpp:436-478) over contiguous inputs.
void broadcast_strides(const int *as, int an, const int *bs, int bn,
                       std::vector<int> &out, std::vector<long> &sa,
                       std::vector<long> &sb) {
  int nd = std::max(an, bn);
  out.assign(nd, 1);
  sa.assign(nd, 0);
  sb.assign(nd, 0);
  std::vector<long> ca(an), cb(bn);
  long s = 1;
  for (int i = an - 1; i >= 0; --i) { ca[i] = s; s *= as[i]; }
  s = 1;
  for (int i = bn - 1; i >= 0; --i) { cb[i] = s; s *= bs[i]; }
  for (int i = 0; i < nd; ++i) {
    int ia = an - 1 - i, ib = bn - 1 - i, o = nd - 1 - i;
    int da = ia >= 0 ? as[ia] : 1, db = ib >= 0 ? bs[ib] : 1;
    if (da != db && da != 1 && db != 1) throw std::runtime_error("broadcast mismatch");
    out[o] = std::max(da, db);
    sa[o] = ia >= 0 ? ((da == 1 && db != 1) ? 0 : ca[ia]) : 0;
    sb[o] = ib >= 0 ? ((db == 1 && da != 1) ? 0 : cb[ib]) : 0;
  }
}

void binary(int dt, int op, const void *a, const int *as, int an, const void *b,
            const int *bs, int bn, void *out) {
  std::vector<int> os;
  std::vector<long> sa, sb;
  broadcast_strides(as, an, bs, bn, os, sa, sb);
  size_t total = 1;
  for (int d : os) total *= size_t(d);
  const int nd = int(os.size());
  par_for(total, [&](size_t s, size_t e) {
    for (size_t i = s; i < e; ++i) {
      size_t offa = 0, offb = 0, cur = i;
      for (int d = nd - 1; d >= 0; --d) {
        size_t c = cur % os[d];
        offa += c * sa[d];
        offb += c * sb[d];
        cur /= os[d];
      }
      if (dt == F32) {
        const float *ap = static_cast<const float *>(a), *bp = static_cast<const float *>(b);
        static_cast<float *>(out)[i] = binop<float>(op, ap[offa], bp[offb]);
      } else {
        wr(out, dt, i, binop<double>(op, rd(a, dt, offa), rd(b, dt, offb)));
      }
    }
  }, dt == F32 ? BACKEND : SERIAL);
}

void relu(int dt, const void *in, void *out, size_t n) {
  par_for(n, [&](size_t s, size_t e) {
    for (size_t i = s; i < e; ++i) {
      if (dt == F32) {
        float x = static_cast<const float *>(in)[i];
        static_cast<float *>(out)[i] = x > 0 ? x : 0;
      } else {
        double v = rd(in, dt, i);
        wr(out, dt, i, std::max(v, 0.0));
      }
    }
  }, dt == F32 ? BACKEND : SERIAL);
}

void sigmoid(int dt, const void *in, void *out, size_t n) {
  par_for(n, [&](size_t s, size_t e) {
    for (size_t i = s; i < e; ++i) {
      if (dt == F32) {
        float x = static_cast<const float *>(in)[i];
        static_cast<float *>(out)[i] = 1.0f / (1.0f + std::exp(-x));
      } else {
        double v = rd(in, dt, i);
        wr(out, dt, i, 1.0 / (1.0 + std::exp(-v)));
      }
    }
  }, dt == F32 ? BACKEND : SERIAL);
}

// nn::GELU (activations.hpp:31-38): c = fill(1.702f) in dtype; x*sigmoid(x*c)
// as three rounded ops with broadcast of the [1] constant.
void gelu(int dt, const void *in, void *out, size_t n) {
  std::vector<uint8_t> cbuf(4), t1(n * dsize(dt)), t2(n * dsize(dt));
  wr(cbuf.data(), dt, 0, double(1.702f));
  int shp[1] = {int(n)}, one[1] = {1};
  binary(dt, MUL, in, shp, 1, cbuf.data(), one, 1, t1.data());
  sigmoid(dt, t1.data(), t2.data(), n);
  binary(dt, MUL, in, shp, 1, t2.data(), shp, 1, out);
}

void softmax(int dt, const void *in, void *out, int rows, int cols) {
  par_for(size_t(rows), [&](size_t s, size_t e) {
    for (size_t r = s; r < e; ++r) {
      size_t base = r * size_t(cols);
      if (dt == F32) {
        const float *x = static_cast<const float *>(in) + base;
        float *y = static_cast<float *>(out) + base;
        float mx = x[0];
        for (int i = 1; i < cols; ++i) if (x[i] > mx) mx = x[i];
        double sum = 0.0;
        for (int i = 0; i < cols; ++i) sum += std::exp(double(x[i]) - double(mx));
        for (int i = 0; i < cols; ++i) y[i] = float(std::exp(double(x[i]) - double(mx)) / sum);
      } else {
        double mx = rd(in, dt, base);
        for (int i = 1; i < cols; ++i) mx = std::max(mx, rd(in, dt, base + i));
        double sum = 0.0;
        for (int i = 0; i < cols; ++i) sum += std::exp(rd(in, dt, base + i) - mx);
        for (int i = 0; i < cols; ++i) wr(out, dt, base + i, std::exp(rd(in, dt, base + i) - mx) / sum);
      }
    }
  }, dt == F32 ? BACKEND : SERIAL);
}

void layer_norm(int dt, const void *x, const void *w, const void *b, void *out,
                int rows, int cols, float eps) {
  par_for(size_t(rows), [&](size_t s, size_t e) {
    for (size_t r = s; r < e; ++r) {
      size_t base = r * size_t(cols);
      double mean = 0.0;
      for (int c = 0; c < cols; ++c) mean += rd(x, dt, base + c);
      mean /= cols;
      double var = 0.0;
      for (int c = 0; c < cols; ++c) {
        double d = rd(x, dt, base + c) - mean;
        var += d * d;
      }
      var /= cols;
      double inv = 1.0 / std::sqrt(var + eps);
      for (int c = 0; c < cols; ++c) {
        double xh = (rd(x, dt, base + c) - mean) * inv;
        wr(out, dt, base + c, xh * rd(w, dt, c) + rd(b, dt, c));
      }
    }
  }, SERIAL);
}

// MultiHeadAttention::forward_impl core (attention.hpp:51-99) from projected
// q2d/k2d/v2d [B*T, E] to the merged context [B*T, E].  The dense [BHT]^2
// mask is block diagonal; masked entries contribute exact zeros to every sum,
// so each (b,h) block is computed on its own with the reference's own
// operation order (documented in the function body).
// textbook: key j of block bh is row bh*T + j of the head-split k (the usual
// attention), instead of the reference's reading of k's buffer as a
// [hd, B*H*T] matrix; every rounding step stays the reference's.  This is the
// attention of the build's autoregressive decode (a KV cache needs each key
// to be its own position's), which MuNet itself does not have.
void mha_core(int dt, const void *q2d, const void *k2d, const void *v2d,
              void *ctx2d, int B, int T, int H, int hd, bool causal, bool textbook) {
  const int E = H * hd, BH = B * H;
  const size_t N = size_t(BH) * T, es = dsize(dt);
  // permute [B,T,H,hd] -> [B,H,T,hd] contiguous (bit copies).
  std::vector<uint8_t> q(N * hd * es), k(N * hd * es), v(N * hd * es);
  for (int bb = 0; bb < B; ++bb)
    for (int t = 0; t < T; ++t)
      for (int h = 0; h < H; ++h) {
        size_t src = (size_t(bb) * T + t) * E + size_t(h) * hd;
        size_t dst = ((size_t(bb) * H + h) * T + t) * hd;
        std::memcpy(q.data() + dst * es, static_cast<const uint8_t *>(q2d) + src * es, hd * es);
        std::memcpy(k.data() + dst * es, static_cast<const uint8_t *>(k2d) + src * es, hd * es);
        std::memcpy(v.data() + dst * es, static_cast<const uint8_t *>(v2d) + src * es, hd * es);
      }
  // scale tensor [1] in dtype (attention.hpp:69-71)
  uint8_t scale_buf[4];
  wr(scale_buf, dt, 0, double(1.0f / std::sqrt(float(hd))));
  const double scale_d = rd(scale_buf, dt, 0);
  const float scale_f = float(scale_d);
  // masked_fill value -1e9 written in dtype (elementwise.cpp:31-34)
  uint8_t fill_buf[4];
  wr(fill_buf, dt, 0, -1e9);
  const double fill_d = rd(fill_buf, dt, 0);

  std::vector<float> qf, kf, vf;
  if (dt == F32 || dt == F16) {
    qf = to_f32(q.data(), dt, N * hd);
    kf = to_f32(k.data(), dt, N * hd);
    vf = to_f32(v.data(), dt, N * hd);
  }
  std::vector<uint8_t> ctx(N * hd * es);
  par_for(size_t(BH) * T, [&](size_t s, size_t e) {
    std::vector<double> row(T);   // scores after scale+mask, in dtype values
    std::vector<double> prob(T);
    for (size_t gi = s; gi < e; ++gi) {
      const size_t bh = gi / T, i = gi % T;
      const size_t col0 = bh * T;
      // scores[gi][col0+j] = sum_k Q[gi][k] * Kflat[k*N + col0 + j]
      // (textbook: K[col0+j][k])
      for (int j = 0; j < T; ++j) {
        double sc;
        auto kidx = [&](int kk) { return textbook ? (col0 + j) * hd + kk : size_t(kk) * N + col0 + j; };
        if (dt == F32 || dt == F16) {
          float sum = 0.0f;
          for (int kk = 0; kk < hd; ++kk)
            sum += qf[gi * hd + kk] * kf[kidx(kk)];
          // matmul output rounded to dtype, then scaled by the [1] tensor
          if (dt == F32) {
            sc = double(sum * scale_f);
          } else {
            double sv = double(dec_f16(enc_f16(sum)));
            uint16_t t = enc_f16(float(sv * scale_d));
            sc = double(dec_f16(t));
          }
        } else {
          double sum = 0.0;
          for (int kk = 0; kk < hd; ++kk)
            sum += rd(q.data(), dt, gi * hd + kk) * rd(k.data(), dt, kidx(kk));
          double sv = double(dec_bf16(enc_bf16(float(sum))));
          sc = double(dec_bf16(enc_bf16(float(sv * scale_d))));
        }
        bool masked = causal && size_t(j) > i;
        row[j] = masked ? fill_d : sc;
      }
      // softmax over the full reference row; entries outside the block are
      // the fill value whose exp underflows to exactly 0 (sum unchanged).
      if (dt == F32) {
        float mx = float(row[0]);
        for (int j = 1; j < T; ++j) if (float(row[j]) > mx) mx = float(row[j]);
        if (BH > 1 && float(fill_d) > mx) mx = float(fill_d);
        double sum = 0.0;
        for (int j = 0; j < T; ++j) sum += std::exp(double(float(row[j])) - double(mx));
        for (int j = 0; j < T; ++j) prob[j] = double(float(std::exp(double(float(row[j])) - double(mx)) / sum));
      } else {
        double mx = row[0];
        for (int j = 1; j < T; ++j) mx = std::max(mx, row[j]);
        if (BH > 1) mx = std::max(mx, fill_d);
        double sum = 0.0;
        for (int j = 0; j < T; ++j) sum += std::exp(row[j] - mx);
        for (int j = 0; j < T; ++j) {
          uint8_t pb[4];
          wr(pb, dt, 0, std::exp(row[j] - mx) / sum);
          prob[j] = rd(pb, dt, 0);
        }
      }
      // ctx = probs @ v (same accumulation type as the matmul path)
      for (int d = 0; d < hd; ++d) {
        if (dt == F32 || dt == F16) {
          float sum = 0.0f;
          for (int j = 0; j < T; ++j) sum += float(prob[j]) * vf[(col0 + j) * hd + d];
          wr(ctx.data(), dt, gi * hd + d, double(sum));
        } else {
          double sum = 0.0;
          for (int j = 0; j < T; ++j) sum += prob[j] * rd(v.data(), dt, (col0 + j) * hd + d);
          wr(ctx.data(), dt, gi * hd + d, sum);
        }
      }
    }
  }, dt == BF16 ? SERIAL : BACKEND);
  // merge heads [B,H,T,hd] -> [B,T,H*hd]
  for (int bb = 0; bb < B; ++bb)
    for (int h = 0; h < H; ++h)
      for (int t = 0; t < T; ++t) {
        size_t src = ((size_t(bb) * H + h) * T + t) * hd;
        size_t dst = (size_t(bb) * T + t) * E + size_t(h) * hd;
        std::memcpy(static_cast<uint8_t *>(ctx2d) + dst * es, ctx.data() + src * es, hd * es);
      }
}

void conv2d(int dt, const void *in, const void *w, const void *bias, void *out,
            int B, int iC, int iH, int iW, int oC, int kH, int kW, int s, int p) {
  const int oH = (iH + 2 * p - kH) / s + 1, oW = (iW + 2 * p - kW) / s + 1;
  std::vector<float> inf, wf, bf;
  const float *ip, *wp, *bp = nullptr;
  if (dt != F32) {
    inf = to_f32(in, dt, size_t(B) * iC * iH * iW);
    wf = to_f32(w, dt, size_t(oC) * iC * kH * kW);
    if (bias) bf = to_f32(bias, dt, oC);
    ip = inf.data(); wp = wf.data(); bp = bias ? bf.data() : nullptr;
  } else {
    ip = static_cast<const float *>(in); wp = static_cast<const float *>(w);
    bp = static_cast<const float *>(bias);
  }
  const size_t total = size_t(B) * oC * oH * oW;
  par_for(total, [&](size_t st, size_t en) {
    for (size_t idx = st; idx < en; ++idx) {
      int ow = int(idx % oW), oh = int((idx / oW) % oH), oc = int((idx / (size_t(oW) * oH)) % oC);
      int b = int(idx / (size_t(oW) * oH * oC));
      float val = bp ? bp[oc] : 0.0f;
      for (int ic = 0; ic < iC; ++ic)
        for (int kh = 0; kh < kH; ++kh)
          for (int kw = 0; kw < kW; ++kw) {
            int ih = oh * s - p + kh, iw = ow * s - p + kw;
            if (ih >= 0 && ih < iH && iw >= 0 && iw < iW)
              val += ip[((size_t(b) * iC + ic) * iH + ih) * iW + iw] *
                     wp[((size_t(oc) * iC + ic) * kH + kh) * kW + kw];
          }
      wr(out, dt, idx, double(val));
    }
  });
}

void max_pool2d(int dt, const void *in, void *out, int B, int C, int iH, int iW,
                int k, int s, int p) {
  const int oH = (iH + 2 * p - k) / s + 1, oW = (iW + 2 * p - k) / s + 1;
  const size_t total = size_t(B) * C * oH * oW;
  par_for(total, [&](size_t st, size_t en) {
    for (size_t idx = st; idx < en; ++idx) {
      int ow = int(idx % oW), oh = int((idx / oW) % oH), c = int((idx / (size_t(oW) * oH)) % C);
      int b = int(idx / (size_t(oW) * oH * C));
      float mx = -1e9f;
      for (int kh = 0; kh < k; ++kh)
        for (int kw = 0; kw < k; ++kw) {
          int ih = oh * s - p + kh, iw = ow * s - p + kw;
          if (ih >= 0 && ih < iH && iw >= 0 && iw < iW)
            mx = std::max(mx, float(rd(in, dt, ((size_t(b) * C + c) * iH + ih) * iW + iw)));
        }
      wr(out, dt, idx, double(mx));
    }
  });
}

} // namespace

#define ORC_GUARD(...)                                                        \
  try {                                                                        \
    __VA_ARGS__;                                                                    \
    return 0;                                                                  \
  } catch (const std::exception &e) {                                          \
    g_err = e.what();                                                          \
    return 1;                                                                  \
  }

extern "C" {

const char *orc_last_error() { return g_err.c_str(); }

// Threads the restatement's parallel loops use (std::thread::hardware_concurrency).
int orc_threads() { return int(std::max(1u, std::thread::hardware_concurrency())); }

// Threading mode of every later call in this process: 0 = parity (split every
// loop over independent outputs), 1 = reference (MuNet's own split, see Path).
int orc_set_threading(int mode) {
  if (mode != 0 && mode != 1) { g_err = "threading mode must be 0 or 1"; return 1; }
  g_threading = mode;
  return 0;
}

int orc_encode(int dt, const float *src, void *dst, size_t n) {
  ORC_GUARD(for (size_t i = 0; i < n; ++i) wr(dst, dt, i, double(src[i])))
}

int orc_decode(int dt, const void *src, float *dst, size_t n) {
  ORC_GUARD(for (size_t i = 0; i < n; ++i) dst[i] = float(rd(src, dt, i)))
}

// Linear/matmul: A [batch*M, K] x B ([K,N] or [batch,K,N]).
int orc_matmul(int dt, const void *a, const void *b, void *out, int batch,
               int M, int K, int N, int b_batched, int transA, int transB) {
  ORC_GUARD(matmul_slices(dt, a, b, out, batch, M, K, N, b_batched != 0,
                          transA != 0, transB != 0))
}

int orc_binary(int dt, int op, const void *a, const int *as, int an,
               const void *b, const int *bs, int bn, void *out) {
  ORC_GUARD(binary(dt, op, a, as, an, b, bs, bn, out))
}

int orc_relu(int dt, const void *in, void *out, size_t n) { ORC_GUARD(relu(dt, in, out, n)) }
int orc_sigmoid(int dt, const void *in, void *out, size_t n) { ORC_GUARD(sigmoid(dt, in, out, n)) }
int orc_gelu(int dt, const void *in, void *out, size_t n) { ORC_GUARD(gelu(dt, in, out, n)) }
int orc_softmax(int dt, const void *in, void *out, int rows, int cols) {
  ORC_GUARD(softmax(dt, in, out, rows, cols))
}
int orc_layer_norm(int dt, const void *x, const void *w, const void *b, void *out,
                   int rows, int cols, float eps) {
  ORC_GUARD(layer_norm(dt, x, w, b, out, rows, cols, eps))
}
int orc_mha_core(int dt, const void *q2d, const void *k2d, const void *v2d,
                 void *ctx, int B, int T, int H, int hd, int causal) {
  ORC_GUARD(mha_core(dt, q2d, k2d, v2d, ctx, B, T, H, hd, causal != 0, false))
}

int orc_mha_core_textbook(int dt, const void *q2d, const void *k2d, const void *v2d,
                          void *ctx, int B, int T, int H, int hd, int causal) {
  ORC_GUARD(mha_core(dt, q2d, k2d, v2d, ctx, B, T, H, hd, causal != 0, true))
}

// Embedding gather (linear.hpp:92-128): ids int32 [n], weight [V, D].
int orc_embedding(int dt, const int32_t *ids, const void *weight, void *out,
                  int n, int V, int D) {
  ORC_GUARD({
    const size_t es = dsize(dt);
    for (int i = 0; i < n; ++i) {
      int tok = ids[i];
      if (tok < 0 || tok >= V) throw std::runtime_error("Embedding index out of range");
      for (int d = 0; d < D; ++d)
        wr(out, dt, size_t(i) * D + d, rd(weight, dt, size_t(tok) * D + d));
    }
    (void)es;
  })
}

int orc_masked_fill(int dt, const void *x, const int32_t *mask, void *out,
                    size_t n, double value) {
  ORC_GUARD(for (size_t i = 0; i < n; ++i) wr(out, dt, i, mask[i] != 0 ? value : rd(x, dt, i)))
}

int orc_conv2d(int dt, const void *in, const void *w, const void *bias,
               void *out, int B, int iC, int iH, int iW, int oC, int kH, int kW,
               int s, int p) {
  ORC_GUARD(conv2d(dt, in, w, bias, out, B, iC, iH, iW, oC, kH, kW, s, p))
}

int orc_max_pool2d(int dt, const void *in, void *out, int B, int C, int iH,
                   int iW, int k, int s, int p) {
  ORC_GUARD(max_pool2d(dt, in, out, B, C, iH, iW, k, s, p))
}

int orc_upsample2d(int dt, const void *in, void *out, int B, int C, int iH,
                   int iW, int scale) {
  ORC_GUARD({
    const int oH = iH * scale, oW = iW * scale;
    const size_t es = dsize(dt);
    for (size_t idx = 0; idx < size_t(B) * C * oH * oW; ++idx) {
      int ow = int(idx % oW), oh = int((idx / oW) % oH);
      size_t bc = idx / (size_t(oW) * oH);
      size_t src = (bc * iH + oh / scale) * iW + ow / scale;
      std::memcpy(static_cast<uint8_t *>(out) + idx * es,
                  static_cast<const uint8_t *>(in) + src * es, es);
    }
  })
}

// Concat of `count` contiguous inputs along `dim` (cpu_backend.hpp:416-452),
// every input sharing rank `ndim`; shapes is count x ndim.
int orc_concat(int dt, const void *const *inputs, const int *shapes, int count,
               int ndim, int dim, void *out) {
  ORC_GUARD({
    const size_t es = dsize(dt);
    size_t outer = 1, inner = 1, total_dim = 0;
    for (int i = 0; i < dim; ++i) outer *= size_t(shapes[i]);
    for (int i = dim + 1; i < ndim; ++i) inner *= size_t(shapes[i]);
    for (int j = 0; j < count; ++j) total_dim += size_t(shapes[j * ndim + dim]);
    for (size_t o = 0; o < outer; ++o) {
      size_t off = o * total_dim * inner;
      for (int j = 0; j < count; ++j) {
        size_t len = size_t(shapes[j * ndim + dim]) * inner;
        std::memcpy(static_cast<uint8_t *>(out) + off * es,
                    static_cast<const uint8_t *>(inputs[j]) + o * len * es, len * es);
        off += len;
      }
    }
  })
}

} // extern "C"
