// Text and base64 forms of embeddings, and the response body around them
// (include/eg2_format.h).
//
// Shortest round-trip float formatting, from the definition: a positive
// float v = m 2^e reads back from every decimal inside its rounding interval
// [v - gap_below / 2, v + gap_above / 2] (the ends included when m is even,
// since reading rounds ties to even), so the shortest such decimal is
// d 10^k for the largest k at which the interval holds a multiple of 10^k,
// and among the multiples at that k the one nearest to v (ties to even d).
// Everything is exact integer arithmetic on the interval in units of
// 2^(e-2): [4m - g, 4m + 2] with g = 2, or g = 1 at the bottom of a binade
// where the gap below is half as wide. The finest step considered, 10^kw,
// is at most half the interval width, so the interval holds a multiple of
// it; coarser steps 10^(kw+j) are then tested on the integer bounds alone.
#include "eg2_format.h"

#include <cmath>
#include <cstdio>
#include <cstring>

#include "eg2_stream.h"

namespace {

typedef unsigned __int128 u128;

constexpr int kEmbd = 768;

// 10^i for i = 0..38 (all below 2^128), built by multiplication.
struct Pow10 {
  u128 p[39];
  Pow10() {
    p[0] = 1;
    for (int i = 1; i < 39; ++i) p[i] = p[i - 1] * 10;
  }
};
const Pow10 kPow10;

// 256-bit unsigned integers for the magnitudes beyond 128 bits
// (subnormals, values near the largest float).
struct U256 {
  uint64_t w[4] = {0, 0, 0, 0};
};
void mul_small(U256& a, uint64_t m) {
  u128 carry = 0;
  for (uint64_t& x : a.w) {
    const u128 p = (u128)x * m + carry;
    x = (uint64_t)p;
    carry = p >> 64;
  }
}
void shl(U256& a, int s) {
  while (s >= 64) {
    a.w[3] = a.w[2];
    a.w[2] = a.w[1];
    a.w[1] = a.w[0];
    a.w[0] = 0;
    s -= 64;
  }
  if (s == 0) return;
  for (int i = 3; i > 0; --i) a.w[i] = (a.w[i] << s) | (a.w[i - 1] >> (64 - s));
  a.w[0] <<= s;
}
void shr1(U256& a) {
  for (int i = 0; i < 3; ++i) a.w[i] = (a.w[i] >> 1) | (a.w[i + 1] << 63);
  a.w[3] >>= 1;
}
int cmp(const U256& a, const U256& b) {
  for (int i = 3; i >= 0; --i)
    if (a.w[i] != b.w[i]) return a.w[i] < b.w[i] ? -1 : 1;
  return 0;
}
void sub(U256& a, const U256& b) {
  uint64_t borrow = 0;
  for (int i = 0; i < 4; ++i) {
    const uint64_t x = a.w[i], y = b.w[i];
    const uint64_t d = x - y - borrow;
    borrow = (x < y) || (x == y && borrow) ? 1 : 0;
    a.w[i] = d;
  }
}
int bits256(const U256& a) {
  for (int i = 3; i >= 0; --i)
    if (a.w[i]) return 64 * i + 64 - __builtin_clzll(a.w[i]);
  return 0;
}

// x 2^E / 10^k: quotient, whether it is exact, and the sign of
// 2 * remainder - denominator (how the fraction compares with one half).
struct Quot {
  uint64_t q;
  bool exact;
  int half;
};

Quot scaled_div(uint64_t x, int E, int k) {
  const int a = E > 0 ? E : 0, c = E < 0 ? -E : 0;  // powers of two above / below
  const int b = k < 0 ? -k : 0, f = k > 0 ? k : 0;  // powers of ten above / below
  // 10^i < 2^(3.33 i): 10 i / 3 + 1 bits.
  if (64 - __builtin_clzll(x) + a + (10 * b) / 3 + 1 <= 127 && c + (10 * f) / 3 + 1 <= 127) {
    const u128 n = ((u128)x << a) * kPow10.p[b];
    const u128 d = ((u128)1 << c) * kPow10.p[f];
    const u128 q = n / d, r = n - q * d;
    const u128 r2 = r << 1;  // r < d < 2^127
    return {(uint64_t)q, r == 0, r2 < d ? -1 : (r2 > d ? 1 : 0)};
  }
  U256 n, d;
  n.w[0] = x;
  shl(n, a);
  for (int i = 0; i < b; ++i) mul_small(n, 10);
  d.w[0] = 1;
  shl(d, c);
  for (int i = 0; i < f; ++i) mul_small(d, 10);
  // Long division; the quotient stays far below 2^63.
  uint64_t q = 0;
  const int s = bits256(n) - bits256(d);
  if (s >= 0) {
    U256 t = d;
    shl(t, s);
    for (int i = s; i >= 0; --i) {
      if (cmp(n, t) >= 0) {
        sub(n, t);
        q |= 1ull << i;
      }
      shr1(t);
    }
  }
  U256 r2 = n;
  shl(r2, 1);
  const int h = cmp(r2, d);
  return {q, bits256(n) == 0, h};
}

uint64_t ceil_div(uint64_t a, uint64_t b) { return a / b + (a % b != 0); }

// float_format.c:244-274 layout of digits d_1..d_len times 10^k.
char* layout(char* p, const char* digits, int len, int k) {
  const int n = len + k;  // position of the decimal point after the digits' start
  if (len <= n && n <= 6) {
    std::memcpy(p, digits, len);
    std::memset(p + len, '0', n - len);
    p += n;
    *p++ = '.';
    *p++ = '0';
    return p;
  }
  if (0 < n && n <= 6) {
    std::memcpy(p, digits, n);
    p[n] = '.';
    std::memcpy(p + n + 1, digits + n, len - n);
    return p + len + 1;
  }
  if (-4 < n && n <= 0) {
    *p++ = '0';
    *p++ = '.';
    std::memset(p, '0', -n);
    p += -n;
    std::memcpy(p, digits, len);
    return p + len;
  }
  *p++ = digits[0];
  if (len > 1) {
    *p++ = '.';
    std::memcpy(p, digits + 1, len - 1);
    p += len - 1;
  }
  *p++ = 'e';
  int x = n - 1;
  *p++ = x < 0 ? '-' : '+';
  if (x < 0) x = -x;
  if (x >= 100) {
    *p++ = (char)('0' + x / 100);
    x %= 100;
  }
  *p++ = (char)('0' + x / 10);
  *p++ = (char)('0' + x % 10);
  return p;
}

void append(char*& p, const char* s) {
  const size_t n = std::strlen(s);
  std::memcpy(p, s, n);
  p += n;
}

}  // namespace

extern "C" size_t eg2_f32_to_chars(char* dst, float value) {
  if (!std::isfinite(value)) return 0;
  char* p = dst;
  if (std::signbit(value)) {
    *p++ = '-';
    value = -value;
  }
  if (value == 0.0f) {
    append(p, "0.0");
    return (size_t)(p - dst);
  }
  uint32_t bits;
  std::memcpy(&bits, &value, 4);
  const uint32_t ef = bits >> 23, frac = bits & 0x7FFFFFu;
  const uint64_t m = ef ? (frac | 0x800000u) : frac;
  const int e = ef ? (int)ef - 150 : -149;
  const uint64_t g = (frac == 0 && ef > 1) ? 1 : 2;
  const uint64_t xl = 4 * m - g, xv = 4 * m, xh = 4 * m + 2;
  const int E = e - 2;
  const bool inclusive = (m & 1) == 0;
  // 10^kw <= half the width (2 + g) 2^E; the estimate may only err low,
  // which costs one more coarsening step.
  const int kw = (int)std::floor(std::log10((double)(2 + g) * 0.5) + E * 0.30102999566398120) - 1;
  const Quot L = scaled_div(xl, E, kw), H = scaled_div(xh, E, kw), V = scaled_div(xv, E, kw);
  const uint64_t dl = inclusive ? L.q + (L.exact ? 0 : 1) : L.q + 1;
  const uint64_t dh = (!inclusive && H.exact) ? H.q - 1 : H.q;
  uint64_t p10 = 1;
  int j = 0;
  while (j < 18 && ceil_div(dl, p10 * 10) <= dh / (p10 * 10)) {
    p10 *= 10;
    ++j;
  }
  // Nearest multiple of 10^(kw + j) to v, ties to even: with v / 10^kw =
  // V.q + frac, the remainder at the coarse step compares with one half as
  // t 10^kw + 2 frac 10^kw, t = 2 (V.q mod 10^j) - 10^j.
  const uint64_t qv = V.q / p10, rv = V.q % p10;
  const int64_t t = 2 * (int64_t)rv - (int64_t)p10;
  int s;
  if (t >= 1) s = 1;
  else if (t <= -2) s = -1;
  else if (t == 0) s = V.exact ? 0 : 1;
  else s = V.half;
  uint64_t d = qv + ((s > 0 || (s == 0 && (qv & 1))) ? 1 : 0);
  const uint64_t lo = ceil_div(dl, p10), hi = dh / p10;
  if (d < lo) d = lo;
  if (d > hi) d = hi;
  char rev[24], digits[24];
  int len = 0;
  for (uint64_t x = d; x; x /= 10) rev[len++] = (char)('0' + x % 10);
  for (int i = 0; i < len; ++i) digits[i] = rev[len - 1 - i];
  return (size_t)(layout(p, digits, len, kw + j) - dst);
}

extern "C" size_t eg2_base64_f32(const float* values, size_t count, char* dst) {
  static const char kAlphabet[] = "ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz0123456789+/";
  const size_t n = 4 * count;
  auto byte = [&](size_t i) -> uint32_t {
    uint32_t w;
    std::memcpy(&w, values + i / 4, 4);
    return (w >> (8 * (i % 4))) & 0xFFu;
  };
  size_t o = 0;
  for (size_t i = 0; i < n; i += 3) {
    const uint32_t b0 = byte(i), b1 = i + 1 < n ? byte(i + 1) : 0, b2 = i + 2 < n ? byte(i + 2) : 0;
    const uint32_t v = (b0 << 16) | (b1 << 8) | b2;
    dst[o++] = kAlphabet[v >> 18];
    dst[o++] = kAlphabet[(v >> 12) & 63];
    dst[o++] = i + 1 < n ? kAlphabet[(v >> 6) & 63] : '=';
    dst[o++] = i + 2 < n ? kAlphabet[v & 63] : '=';
  }
  return o;
}

extern "C" size_t eg2_embeddings_response_bound(size_t n, unsigned dims, size_t model_len) {
  // Per value at most 32 characters + a comma (or 6 base64 characters);
  // per embedding the wrapper and index; the model name at most 6 bytes per
  // byte escaped.
  return n * ((size_t)dims * 33 + 96) + 6 * model_len + 256;
}

extern "C" size_t eg2_embeddings_response(float* embeddings, size_t n, unsigned dims, eg2_embedding_api api,
                                          eg2_embedding_encoding encoding, const char* model, size_t model_len,
                                          size_t prompt_tokens, char* dst, size_t cap) {
  if (!embeddings || !dst || (model_len && !model)) return 0;
  if (dims != 128 && dims != 256 && dims != 512 && dims != (unsigned)kEmbd) return 0;
  if (cap < eg2_embeddings_response_bound(n, dims, model_len)) return 0;
  const bool openai = api == EG2_API_OPENAI;
  char* p = dst;
  append(p, openai ? "{\"object\":\"list\",\"data\":[" : "{\"embeddings\":[");
  for (size_t i = 0; i < n; ++i) {
    float* e = embeddings + i * kEmbd;
    if (!eg2_normalize_prefix(e, dims)) return 0;
    if (i) *p++ = ',';
    if (openai) append(p, "{\"object\":\"embedding\",\"embedding\":");
    if (encoding == EG2_ENCODING_BASE64) {
      *p++ = '"';
      p += eg2_base64_f32(e, dims, p);
      *p++ = '"';
    } else {
      *p++ = '[';
      for (unsigned d = 0; d < dims; ++d) {
        if (d) *p++ = ',';
        const size_t w = eg2_f32_to_chars(p, e[d]);
        if (!w) return 0;
        p += w;
      }
      *p++ = ']';
    }
    if (openai) p += std::snprintf(p, 64, ",\"index\":%zu}", i);
  }
  if (openai) {
    append(p, "],\"model\":\"");
    for (size_t i = 0; i < model_len; ++i) {
      const unsigned char c = (unsigned char)model[i];
      switch (c) {
        case '"': append(p, "\\\""); break;
        case '\\': append(p, "\\\\"); break;
        case '\b': append(p, "\\b"); break;
        case '\f': append(p, "\\f"); break;
        case '\n': append(p, "\\n"); break;
        case '\r': append(p, "\\r"); break;
        case '\t': append(p, "\\t"); break;
        default:
          if (c < 0x20) p += std::snprintf(p, 8, "\\u%04x", c);
          else *p++ = (char)c;
      }
    }
    p += std::snprintf(p, 160, "\",\"usage\":{\"prompt_tokens\":%zu,\"total_tokens\":%zu}}", prompt_tokens,
                       prompt_tokens);
  } else {
    append(p, "]}");
  }
  *p = '\0';
  return (size_t)(p - dst);
}
