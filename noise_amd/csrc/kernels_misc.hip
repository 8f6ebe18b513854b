// Stand-alone entry points over the shared kernels: the windowed attention forward and the credit passes.
#include <string.h>

#include "window_flash.h"

using namespace noise;

extern "C" int noise_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t batch, int32_t heads,
                               int64_t T, int64_t stride_b, int64_t stride_t, int32_t window, uint16_t* out,
                               int64_t out_stride_b, int64_t out_stride_t, float* lse, void* stream) {
  NOISE_REQUIRE(q && k && v && out, "NULL pointer argument");
  NOISE_REQUIRE(batch > 0 && batch <= 65535 && heads > 0 && heads <= 65535, "batch / heads outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  NOISE_REQUIRE(stride_t % 8 == 0 && stride_b % 8 == 0 && out_stride_t % 4 == 0, "strides must keep 16-byte rows");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = q; a.y = k; a.v = v;
  a.x_sb = a.y_sb = a.v_sb = stride_b;
  a.x_st = a.y_st = a.v_st = stride_t;
  a.out = out; a.o_sb = out_stride_b; a.o_st = out_stride_t;
  a.lse_out = lse;
  a.heads = heads; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeAttention, (hipStream_t)stream);
  NOISE_CHECK_HIP((launch_flash<kAttn, false, 1>(a, batch, heads, (hipStream_t)stream)));
  return NOISE_OK;
}

extern "C" int noise_attention_periodic(const uint16_t* q, int32_t q_period, const uint16_t* k, int32_t k_period,
                                        const uint16_t* v, int32_t v_period, int64_t batch, int32_t heads, int64_t T,
                                        int64_t stride_b, int64_t stride_t, int32_t window, int32_t bounded,
                                        uint16_t* out, int64_t out_stride_b, int64_t out_stride_t, void* stream) {
  NOISE_REQUIRE(q && k && v && out, "NULL pointer argument");
  NOISE_REQUIRE(batch > 0 && batch <= 65535 && heads > 0 && heads <= 65535, "batch / heads outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  NOISE_REQUIRE(q_period >= 0 && k_period >= 0 && v_period >= 0, "negative period");
  NOISE_REQUIRE(stride_t % 8 == 0 && stride_b % 8 == 0 && out_stride_t % 4 == 0, "strides must keep 16-byte rows");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = q; a.y = k; a.v = v;
  a.x_sb = a.y_sb = a.v_sb = stride_b;
  a.x_st = a.y_st = a.v_st = stride_t;
  a.x_period = q_period; a.y_period = k_period; a.v_period = v_period;
  a.out = out; a.o_sb = out_stride_b; a.o_st = out_stride_t;
  a.heads = heads; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeAttention, (hipStream_t)stream);
  if (bounded)
    NOISE_CHECK_HIP((launch_flash<kAttn, true, 1>(a, batch, heads, (hipStream_t)stream)));  // |q . k| / 8 <= 8
  else
    NOISE_CHECK_HIP((launch_flash<kAttn, false, 1>(a, batch, heads, (hipStream_t)stream)));
  return NOISE_OK;
}

extern "C" int noise_credit_lse(const uint16_t* q, const uint16_t* k, int64_t rows, int64_t T, int32_t window,
                                float* lse, void* stream) {
  NOISE_REQUIRE(q && k && lse, "NULL pointer argument");
  NOISE_REQUIRE(rows > 0 && rows <= 65535, "rows outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = q; a.y = k;
  a.x_sb = a.y_sb = T * 64; a.x_st = a.y_st = 64;
  a.lse_out = lse;
  a.heads = 1; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeCreditLse, (hipStream_t)stream);
  NOISE_CHECK_HIP((launch_flash<kLse, false, 1>(a, rows, 1, (hipStream_t)stream)));
  return NOISE_OK;
}

extern "C" int noise_credit_lse_bounded(const uint16_t* q, const uint16_t* k, int64_t rows, int64_t T, int32_t window,
                                        float* lse, void* stream) {
  NOISE_REQUIRE(q && k && lse, "NULL pointer argument");
  NOISE_REQUIRE(rows > 0 && rows <= 65535, "rows outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = q; a.y = k;
  a.x_sb = a.y_sb = T * 64; a.x_st = a.y_st = 64;
  a.lse_out = lse;
  a.heads = 1; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeCreditLse, (hipStream_t)stream);
  NOISE_CHECK_HIP((launch_flash<kLse, true, 1>(a, rows, 1, (hipStream_t)stream)));  // the caller's |q . k| / 8 <= 16
  return NOISE_OK;
}

extern "C" int noise_credit_key_context(const uint16_t* q, const uint16_t* k, const uint16_t* values,
                                        const uint16_t* hub, int64_t rows, int64_t T, int32_t window, float* lse,
                                        float* center, void* stream) {
  NOISE_REQUIRE(q && k && values && hub && lse && center, "NULL pointer argument");
  NOISE_REQUIRE(rows > 0 && rows <= 65535, "rows outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = q; a.y = k; a.v = values; a.hub = hub;
  a.x_sb = a.y_sb = a.v_sb = T * 64; a.x_st = a.y_st = a.v_st = 64;
  a.lse_out = lse; a.center_out = center;
  a.heads = 1; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeCreditCenter, (hipStream_t)stream);
  NOISE_CHECK_HIP((launch_flash<kCenter, false, 1>(a, rows, 1, (hipStream_t)stream)));
  return NOISE_OK;
}

extern "C" int noise_credit_value(const uint16_t* q, const uint16_t* k, const float* lse, const float* src, int64_t rows,
                                  int64_t T, int32_t window, int32_t hi_lo, float* out, void* stream) {
  NOISE_REQUIRE(q && k && lse && src && out, "NULL pointer argument");
  NOISE_REQUIRE(rows > 0 && rows <= 65535, "rows outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = k; a.y = q; a.v = src;
  a.x_sb = a.y_sb = a.v_sb = T * 64; a.x_st = a.y_st = a.v_st = 64;
  a.lse_in = lse;
  a.out = out; a.o_sb = T * 64; a.o_st = 64;
  a.heads = 1; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeCreditValue, (hipStream_t)stream);
  if (hi_lo)
    NOISE_CHECK_HIP((launch_flash<kCredit, true, 1>(a, rows, 1, (hipStream_t)stream)));
  else
    NOISE_CHECK_HIP((launch_flash<kCredit, false, 1>(a, rows, 1, (hipStream_t)stream)));
  return NOISE_OK;
}

extern "C" int noise_credit_value_strided(const uint16_t* q, const uint16_t* k, const float* lse, const float* src,
                                          int32_t src_heads, int64_t src_sb, int64_t src_st, int64_t rows, int64_t T,
                                          int32_t window, int32_t hi_lo, float* out, int32_t out_heads, int64_t out_sb,
                                          int64_t out_st, const int32_t* out_rows, void* stream) {
  NOISE_REQUIRE(q && k && lse && src && out, "NULL pointer argument");
  NOISE_REQUIRE(rows > 0 && rows <= 65535, "rows outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  NOISE_REQUIRE(src_heads > 0 && rows % src_heads == 0 && out_heads > 0 && rows % out_heads == 0,
                "rows %lld must divide by src_heads %d and out_heads %d", (long long)rows, src_heads, out_heads);
  NOISE_REQUIRE(src_st >= (int64_t)src_heads * 64 && src_sb >= (T - 1) * src_st + (int64_t)src_heads * 64,
                "source strides (%lld, %lld) too short for %d heads of 64 over T = %lld", (long long)src_sb,
                (long long)src_st, src_heads, (long long)T);
  NOISE_REQUIRE(out_st >= (int64_t)out_heads * 64 && out_sb >= (T - 1) * out_st + (int64_t)out_heads * 64,
                "output strides (%lld, %lld) too short for %d heads of 64 over T = %lld", (long long)out_sb,
                (long long)out_st, out_heads, (long long)T);
  NOISE_REQUIRE(src_st % 4 == 0 && out_st % 4 == 0 && src_sb % 4 == 0 && out_sb % 4 == 0,
                "strides must be multiples of 4 elements (16-byte rows)");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = k; a.y = q; a.v = src;
  a.x_sb = a.y_sb = T * 64; a.x_st = a.y_st = 64;
  a.v_sb = src_sb; a.v_st = src_st; a.v_div = src_heads;
  a.lse_in = lse;
  a.out = out; a.o_sb = out_sb; a.o_st = out_st; a.o_div = out_heads; a.o_map = out_rows;
  a.heads = 1; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeCreditValue, (hipStream_t)stream);
  if (hi_lo)
    NOISE_CHECK_HIP((launch_flash<kCredit, true, 1>(a, rows, 1, (hipStream_t)stream)));
  else
    NOISE_CHECK_HIP((launch_flash<kCredit, false, 1>(a, rows, 1, (hipStream_t)stream)));
  return NOISE_OK;
}
