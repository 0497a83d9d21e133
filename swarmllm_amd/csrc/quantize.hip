// quantize.hip — activation quantizers (bit-exact to candle's from_float),
// on-device weight quantizers (QTensor::quantize) and dequantizers.
//
// Built with -ffp-contract=off: the reference (Rust) never fuses a*b+c, and
// every code and scale produced here must match it bit for bit. Division
// and sqrt are IEEE correctly rounded (hipcc's default for f32).
//
// Reference (vendor/candle/candle-core/src/quantized/, "Q/"):
//   BlockQ8K::from_float  Q/k_quants.rs:2882-2927
//   BlockQ8_0::from_float Q/k_quants.rs:1240-1269
//   BlockQ4K::from_float  Q/k_quants.rs:2113-2171, make_qkx1_quants Q/utils.rs:227-285
//   BlockQ6K::from_float  Q/k_quants.rs:2657-2727, make_qx_quants Q/utils.rs:62-225
//   BlockMxfp4::from_float Q/k_quants.rs:483-506
//   BlockIq4Nl::from_float Q/k_quants.rs:605-701, 727-743
//   to_float per type      Q/k_quants.rs:1222 (Q8_0), 2238 (Q4_K), 2810 (Q6_K), 465 (MXFP4), 709 (IQ4_NL)
#include "qmm_device.h"
#include "qmm_launch.h"
#include "moe_runs.h"

namespace qmm {

// ===========================================================================
// activation layouts
// ===========================================================================
size_t act_bytes(int layout, int64_t k, int64_t rows) {
  const size_t codes = align_up((size_t)(rows * k), 256);
  if (layout == ACT_Q8K) {
    const size_t d = align_up((size_t)(rows * (k / 256)) * 4, 256);
    const size_t bs = align_up((size_t)(rows * (k / 16)) * 2, 256);
    return codes + d + bs;
  }
  const size_t d = align_up((size_t)(rows * (k / 32)) * 4, 256);
  const size_t sums = align_up((size_t)(rows * (k / 32)) * 4, 256);
  return codes + d + sums;
}

void act_plane_offsets(int layout, int64_t k, int64_t rows, size_t* scales_off, size_t* sums_off) {
  const size_t codes = align_up((size_t)(rows * k), 256);
  *scales_off = codes;
  *sums_off = codes + align_up((size_t)(rows * (k / (layout == ACT_Q8K ? 256 : 32))) * 4, 256);
}

ActPlanes act_planes(int layout, void* base, int64_t k, int64_t rows) {
  size_t so = 0, uo = 0;
  act_plane_offsets(layout, k, rows, &so, &uo);
  char* b = (char*)base;
  ActPlanes p;
  p.codes = (int8_t*)b;
  p.d = (float*)(b + so);
  p.sums = (void*)(b + uo);
  return p;
}

ActPlanes act_rows(int layout, const ActPlanes& p, int64_t k, int64_t r0) {
  ActPlanes o;
  o.codes = p.codes + r0 * k;
  if (layout == ACT_Q8K) {
    o.d = p.d + r0 * (k / 256);
    o.sums = (int16_t*)p.sums + r0 * (k / 16);
  } else {
    o.d = p.d + r0 * (k / 32);
    o.sums = (int32_t*)p.sums + r0 * (k / 32);
  }
  return o;
}

// ===========================================================================
// Q8_K activation (per 256): 16 lanes per block (16 values per lane), four
// blocks per wave, through q8k_block_group16 (the routine the fused decode
// kernels run in LDS).
// ===========================================================================
template <bool kVec, bool kRuns = false>
__global__ __launch_bounds__(256) void act_q8k_kernel(const float* __restrict__ x, int64_t stride, int64_t k,
                                                      int64_t rows, int8_t* __restrict__ codes,
                                                      float* __restrict__ dout, int16_t* __restrict__ bsout,
                                                      float qmax, const int32_t* __restrict__ expert_ids = nullptr,
                                                      int size_m = 0, int32_t* __restrict__ runs = nullptr) {
  if (kRuns && blockIdx.x == gridDim.x - 1) {
    moe_runs_block<256>(expert_ids, size_m, runs);
    return;
  }
  const int lane = threadIdx.x & 63, gl = lane & 15;
  const int64_t nbk = k / 256;
  const int64_t blk = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  const bool valid = blk < rows * nbk;  // every lane takes part in the shuffles
  const int64_t bb = valid ? blk : 0;
  const int64_t r = bb / nbk, b = bb - r * nbk;
  const float* xp = x + r * stride + b * 256 + 16 * gl;
  float v[16];
  if (kVec) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 t = ((const float4*)xp)[i];
      v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = xp[i];
  }
  uint32_t c[4];
  int32_t sum16;
  float d;
  q8k_block_group16(v, gl, qmax, c, sum16, d);
  if (!valid) return;
  *(uint4*)(codes + r * k + b * 256 + 16 * gl) = make_uint4(c[0], c[1], c[2], c[3]);
  bsout[r * (k / 16) + b * 16 + gl] = (int16_t)sum16;
  if (gl == 0) dout[r * nbk + b] = d;
}

// ===========================================================================
// Q8_0 activation (per 32), planes: 8 lanes per block, 4 values per lane.
// Also the GGUF-layout Q8_0 weight quantizer (the same from_float).
// ===========================================================================
// kRuns: the last workgroup of the grid writes a grouped expert product's
// run table instead (moe_runs.h), so that product needs no launch of its own
// before the grouped kernel.
template <bool kVec, bool kGguf, bool kRuns = false>
__global__ __launch_bounds__(256) void q8_0_kernel(const float* __restrict__ x, int64_t stride, int64_t k,
                                                   int64_t rows, int8_t* __restrict__ codes,
                                                   float* __restrict__ dout, int32_t* __restrict__ sout,
                                                   uint8_t* __restrict__ gguf,
                                                   const int32_t* __restrict__ expert_ids = nullptr,
                                                   int size_m = 0, int32_t* __restrict__ runs = nullptr) {
  if (kRuns && blockIdx.x == gridDim.x - 1) {
    moe_runs_block<256>(expert_ids, size_m, runs);
    return;
  }
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int sub = (int)(gid & 7);
  const int64_t blk = gid >> 3;
  const int64_t nb = k / 32;
  if (blk >= rows * nb) return;  // whole 8-lane groups
  const int64_t r = blk / nb, b = blk - r * nb;
  const float* xp = x + r * stride + b * 32 + 4 * sub;
  float v[4];
  if (kVec) {
    const float4 t = *(const float4*)xp;
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = xp[i];
  }
  // amax as f32::max folds it (fmaxf ignores NaN the same way); >= 0, so
  // the 8-lane maximum is taken on its bits
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  uint32_t ab = __float_as_uint(fmaxf(amax, 0.0f));
  ab = max(ab, (uint32_t)__shfl_xor((int)ab, 1, kWave));
  ab = max(ab, (uint32_t)__shfl_xor((int)ab, 2, kWave));
  ab = max(ab, (uint32_t)__shfl_xor((int)ab, 4, kWave));
  amax = __uint_as_float(ab);
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const int32_t packed =
      (int32_t)pack4_i8(q8_0_code(v[0] * id), q8_0_code(v[1] * id), q8_0_code(v[2] * id), q8_0_code(v[3] * id));
  int32_t s = __builtin_amdgcn_sdot4(packed, 0x01010101, 0, false);
  const uint16_t dh = f2h(d);
  if (kGguf) {
    uint8_t* o = gguf + blk * 34;
    ((uint16_t*)(o + 2 + 4 * sub))[0] = (uint16_t)(packed & 0xFFFF);
    ((uint16_t*)(o + 2 + 4 * sub))[1] = (uint16_t)((uint32_t)packed >> 16);
    if (sub == 0) *(uint16_t*)o = dh;
  } else {
    s += __shfl_xor(s, 1, kWave);
    s += __shfl_xor(s, 2, kWave);
    s += __shfl_xor(s, 4, kWave);
    ((int32_t*)(codes + r * k + b * 32))[sub] = packed;
    if (sub == 0) {
      dout[r * nb + b] = h2f(dh);
      sout[r * nb + b] = s;
    }
  }
}

hipError_t launch_act_quantize_moe(int layout, const float* x, int64_t stride, int64_t k, int64_t rows, void* out,
                                   const int32_t* expert_ids, int64_t size_m, int32_t* runs, float q8k_scale,
                                   hipStream_t st) {
  const ActPlanes p = act_planes(layout, out, k, rows);
  const bool vec = ((uintptr_t)x % 16 == 0) && (stride % 4 == 0);
  if (layout == ACT_Q8K) {
    const int64_t blocks = rows * (k / 256);
    const dim3 grid((unsigned)((blocks + 15) / 16 + 1));  // + the run table's workgroup
    if (vec)
      act_q8k_kernel<true, true><<<grid, 256, 0, st>>>(x, stride, k, rows, p.codes, p.d, (int16_t*)p.sums, q8k_scale,
                                                       expert_ids, (int)size_m, runs);
    else
      act_q8k_kernel<false, true><<<grid, 256, 0, st>>>(x, stride, k, rows, p.codes, p.d, (int16_t*)p.sums, q8k_scale,
                                                        expert_ids, (int)size_m, runs);
    return hipGetLastError();
  }
  const int64_t threads = rows * (k / 32) * 8;
  const dim3 grid((unsigned)((threads + 255) / 256 + 1));  // + the run table's workgroup
  if (vec)
    q8_0_kernel<true, false, true><<<grid, 256, 0, st>>>(x, stride, k, rows, p.codes, p.d, (int32_t*)p.sums, nullptr,
                                                         expert_ids, (int)size_m, runs);
  else
    q8_0_kernel<false, false, true><<<grid, 256, 0, st>>>(x, stride, k, rows, p.codes, p.d, (int32_t*)p.sums, nullptr,
                                                          expert_ids, (int)size_m, runs);
  return hipGetLastError();
}

hipError_t launch_act_quantize(int layout, const float* x, int64_t stride, int64_t k, int64_t rows, void* out,
                               float q8k_scale, hipStream_t st) {
  const ActPlanes p = act_planes(layout, out, k, rows);
  const bool vec = ((uintptr_t)x % 16 == 0) && (stride % 4 == 0);
  if (layout == ACT_Q8K) {
    const int64_t blocks = rows * (k / 256);
    const dim3 grid((unsigned)((blocks + 15) / 16));
    if (vec)
      act_q8k_kernel<true><<<grid, 256, 0, st>>>(x, stride, k, rows, p.codes, p.d, (int16_t*)p.sums, q8k_scale);
    else
      act_q8k_kernel<false><<<grid, 256, 0, st>>>(x, stride, k, rows, p.codes, p.d, (int16_t*)p.sums, q8k_scale);
  } else {
    const int64_t threads = rows * (k / 32) * 8;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (vec)
      q8_0_kernel<true, false><<<grid, 256, 0, st>>>(x, stride, k, rows, p.codes, p.d, (int32_t*)p.sums, nullptr);
    else
      q8_0_kernel<false, false><<<grid, 256, 0, st>>>(x, stride, k, rows, p.codes, p.d, (int32_t*)p.sums, nullptr);
  }
  return hipGetLastError();
}

// ===========================================================================
// Q4_K weight quantizer: one thread per super-block.
// ===========================================================================
__device__ __forceinline__ int32_t total_key(float f) {
  int32_t i = __builtin_bit_cast(int32_t, f);
  return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

// make_qkx1_quants(nmax = 15, ntry = 5) over 32 values -> (scale, -min).
__device__ void make_qkx1_15_5(const float* __restrict__ xg, float& scale_out, float& negmin_out) {
  float x[32];
#pragma unroll
  for (int i = 0; i < 32; i++) x[i] = xg[i];
  float mn = x[0], mx = x[0];
  int32_t kmn = total_key(x[0]), kmx = kmn;
#pragma unroll
  for (int i = 1; i < 32; i++) {
    const int32_t kk = total_key(x[i]);
    if (kk < kmn) { kmn = kk; mn = x[i]; }
    if (kk >= kmx) { kmx = kk; mx = x[i]; }
  }
  if (mx == mn) { scale_out = 0.0f; negmin_out = 0.0f; return; }
  mn = rs_min(mn, 0.0f);
  float iscale = 15.0f / (mx - mn);
  float scale = 1.0f / iscale;
  int l[32];
#pragma unroll
  for (int i = 0; i < 32; i++) l[i] = 0;
  for (int itry = 0; itry < 5; itry++) {
    float sumlx = 0.0f;
    int32_t suml2 = 0;
    bool changed = false;
#pragma unroll
    for (int i = 0; i < 32; i++) {
      const int li = clampi(nearest_int(iscale * (x[i] - mn)), 0, 15);
      if (li != l[i]) { l[i] = li; changed = true; }
      sumlx += (x[i] - mn) * (float)li;
      suml2 += li * li;
    }
    scale = sumlx / (float)suml2;
    float sum = -0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) sum += x[i] - scale * (float)l[i];
    mn = sum / 32.0f;
    if (mn > 0.0f) mn = 0.0f;
    iscale = 1.0f / scale;
    if (!changed) break;
  }
  scale_out = scale;
  negmin_out = -mn;
}

__global__ __launch_bounds__(256) void quant_q4k_kernel(const float* __restrict__ xall, uint8_t* __restrict__ out,
                                                        int64_t nb) {
  const int64_t ib = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (ib >= nb) return;
  const float* x = xall + ib * 256;
  float scales[8], mins[8];
  for (int j = 0; j < 8; j++) make_qkx1_15_5(x + 32 * j, scales[j], mins[j]);
  float max_scale = 0.0f, max_min = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) max_scale = rs_max(scales[j], max_scale);
#pragma unroll
  for (int j = 0; j < 8; j++) max_min = rs_max(mins[j], max_min);
  const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
  const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
  uint8_t sc[12];
#pragma unroll
  for (int i = 0; i < 12; i++) sc[i] = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int lsi = nearest_int(inv_scale * scales[j]);
    const int lmi = nearest_int(inv_min * mins[j]);
    const uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
    const uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
    if (j < 4) {
      sc[j] = ls;
      sc[j + 4] = lm;
    } else {
      sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
      sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
      sc[j] |= (uint8_t)((lm >> 4) << 6);
    }
  }
  const uint16_t dh = f2h(max_scale / 63.0f), mh = f2h(max_min / 63.0f);
  uint8_t* o = out + ib * 144;
  *(uint32_t*)o = (uint32_t)dh | ((uint32_t)mh << 16);
#pragma unroll
  for (int i = 0; i < 3; i++)
    ((uint32_t*)(o + 4))[i] = (uint32_t)sc[4 * i] | ((uint32_t)sc[4 * i + 1] << 8) |
                              ((uint32_t)sc[4 * i + 2] << 16) | ((uint32_t)sc[4 * i + 3] << 24);
  const float df = h2f(dh), mf = h2f(mh);
  // codes: sub-block j = 2c (low nibbles) and 2c+1 (high nibbles) of chunk c
  for (int c = 0; c < 4; c++) {
    int sc0, m0, sc1, m1;
    scale_min_k4(2 * c, sc, sc0, m0);
    scale_min_k4(2 * c + 1, sc, sc1, m1);
    const float d0 = df * (float)sc0, d1 = df * (float)sc1;
    const float dm0 = mf * (float)m0, dm1 = mf * (float)m1;
    for (int w = 0; w < 8; w++) {
      uint32_t word = 0;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int l = 4 * w + t;
        int lo = 0, hi = 0;
        if (d0 != 0.0f) lo = clampi(nearest_int((x[64 * c + l] + dm0) / d0), 0, 15);
        if (d1 != 0.0f) hi = clampi(nearest_int((x[64 * c + 32 + l] + dm1) / d1), 0, 15);
        word |= (uint32_t)(lo | (hi << 4)) << (8 * t);
      }
      ((uint32_t*)(o + 16 + 32 * c))[w] = word;
    }
  }
}

// ===========================================================================
// Q6_K weight quantizer: one thread per super-block.
// ===========================================================================
// make_qx_quants(n = 16, nmax = 32, rmse_type = 1, weights = x*x).
__device__ float make_qx_16_32(const float* __restrict__ xg, int8_t* L) {
  float x[16];
#pragma unroll
  for (int i = 0; i < 16; i++) x[i] = xg[i];
  const int nmax = 32;
  float max = 0.0f, amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const float ax = fabsf(x[i]);
    if (ax > amax) { amax = ax; max = x[i]; }
  }
  if (amax == 0.0f) {
#pragma unroll
    for (int i = 0; i < 16; i++) L[i] = 0;
    return 0.0f;
  }
  const float iscale0 = -(float)nmax / max;
  float sumlx = 0.0f, suml2 = 0.0f;
  int ls[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int l = clampi(nearest_int(iscale0 * x[i]), -nmax, nmax - 1);
    ls[i] = l + nmax;
    const float w = x[i] * x[i];
    const float lf = (float)l;
    sumlx += w * x[i] * lf;
    suml2 += w * lf * lf;
  }
  float scale = sumlx / suml2;
  float best = scale * sumlx;
  for (int itry = 0; itry < 3; itry++) {
    const float is2 = 1.0f / scale;
    float slx = 0.0f, sl2 = 0.0f;
    bool changed = false;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int l = clampi(nearest_int(is2 * x[i]), -nmax, nmax - 1);
      if (l + nmax != ls[i]) changed = true;
      const float w = x[i] * x[i];
      const float lf = (float)l;
      slx += w * x[i] * lf;
      sl2 += w * lf * lf;
    }
    if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
#pragma unroll
    for (int i = 0; i < 16; i++) ls[i] = nmax + clampi(nearest_int(is2 * x[i]), -nmax, nmax - 1);
    sumlx = slx;
    suml2 = sl2;
    scale = sumlx / suml2;
    best = scale * sumlx;
  }
  for (int itry = 0; itry < 5; itry++) {
    int n_changed = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float w = x[i] * x[i];
      const int l = ls[i] - nmax;
      float slx = sumlx - w * x[i] * (float)l;
      if (slx > 0.0f) {
        float sl2 = suml2 - w * (float)l * (float)l;
        const int new_l = clampi(nearest_int(x[i] * sl2 / slx), -nmax, nmax - 1);
        if (new_l != l) {
          slx += w * x[i] * (float)new_l;
          sl2 += w * (float)new_l * (float)new_l;
          if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
            ls[i] = nmax + new_l;
            sumlx = slx;
            suml2 = sl2;
            scale = sumlx / suml2;
            best = scale * sumlx;
            n_changed++;
          }
        }
      }
    }
    if (n_changed == 0) break;
  }
#pragma unroll
  for (int i = 0; i < 16; i++) L[i] = (int8_t)ls[i];
  return scale;
}

__global__ __launch_bounds__(128) void quant_q6k_kernel(const float* __restrict__ xall, uint8_t* __restrict__ out,
                                                        int64_t nb) {
  const int64_t ib = (int64_t)blockIdx.x * 128 + threadIdx.x;
  if (ib >= nb) return;
  const float* x = xall + ib * 256;
  int8_t L[256];
  float scales[16];
  float max_scale = 0.0f, max_abs_scale = 0.0f;
  for (int g = 0; g < 16; g++) {
    const float s = make_qx_16_32(x + 16 * g, L + 16 * g);
    scales[g] = s;
    const float as = fabsf(s);
    if (as > max_abs_scale) { max_abs_scale = as; max_scale = s; }
  }
  const float iscale = -128.0f / max_scale;
  const uint16_t dh = f2h(1.0f / iscale);
  int8_t ysc[16];
  for (int g = 0; g < 16; g++) {
    const int v = nearest_int(iscale * scales[g]);
    ysc[g] = (int8_t)(v < 127 ? v : 127);
  }
  const float df = h2f(dh);
  for (int j = 0; j < 16; j++) {
    const float d = df * (float)ysc[j];
    if (d == 0.0f) continue;
    for (int ii = 0; ii < 16; ii++) L[16 * j + ii] = (int8_t)(clampi(nearest_int(x[16 * j + ii] / d), -32, 31) + 32);
  }
  uint8_t* o = out + ib * 210;  // 2-byte aligned: write bytes
  for (int j = 0; j < 256; j += 128) {
    uint8_t* ql = o + j / 2;
    uint8_t* qh = o + 128 + j / 4;
    for (int l = 0; l < 32; l++) {
      const uint8_t q1 = (uint8_t)(L[j + l] & 0xF), q2 = (uint8_t)(L[j + l + 32] & 0xF);
      const uint8_t q3 = (uint8_t)(L[j + l + 64] & 0xF), q4 = (uint8_t)(L[j + l + 96] & 0xF);
      ql[l] = (uint8_t)(q1 | (q3 << 4));
      ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
      qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                        ((L[j + l + 96] >> 4) << 6));
    }
  }
  for (int g = 0; g < 16; g++) o[192 + g] = (uint8_t)ysc[g];
  o[208] = (uint8_t)(dh & 0xFF);
  o[209] = (uint8_t)(dh >> 8);
}

// ===========================================================================
// MXFP4 weight quantizer: one thread per 32-block. The exponent is
// floor(log2f(amax)); floor((float)log2((double)amax)) equals glibc's
// floor(log2f(amax)) for every positive finite f32 (checked exhaustively
// over the values where the two could part: within 2^20 ulps of each power
// of two, and all subnormals).
// ===========================================================================
__device__ __forceinline__ uint32_t mxfp4_best_index(float x, float d) {
  uint32_t best = 0;
  float best_err = fabsf((float)kMxfp4Values[0] * d - x);
#pragma unroll
  for (int i = 1; i < 16; i++) {
    const float err = fabsf((float)kMxfp4Values[i] * d - x);
    if (err < best_err) { best = (uint32_t)i; best_err = err; }
  }
  return best;
}

__global__ __launch_bounds__(256) void quant_mxfp4_kernel(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                          int64_t nb) {
  const int64_t ib = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (ib >= nb) return;
  const float* xs = x + ib * 32;
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) {
    const float a = fabsf(xs[j]);
    if (amax < a) amax = a;
  }
  uint32_t e = 0;
  if (amax > 0.0f) e = rs_as_u8(floorf((float)log2((double)amax)) - 2.0f + 127.0f);
  const float d = e8m0_half(e);
  uint8_t* o = out + ib * 17;
  o[0] = (uint8_t)e;
  for (int j = 0; j < 16; j++) o[1 + j] = (uint8_t)(mxfp4_best_index(xs[j], d) | (mxfp4_best_index(xs[16 + j], d) << 4));
}

// ===========================================================================
// IQ4_NL weight quantizer. A block whose values are all below 1e-15 in
// magnitude keeps the levels of the last block before it that had any (the
// reference carries its levels array from block to block), so the blocks
// are done in two passes: each block alone, then a scan that hands a
// "zero" block the codes of the nearest earlier non-zero block.
// ===========================================================================
__device__ __forceinline__ uint32_t iq4_best_index(float x) {
  if (x <= (float)kIq4nlValues[0]) return 0;
  if (x >= (float)kIq4nlValues[15]) return 15;
  int ml = 0, mu = 15;
  while (mu - ml > 1) {
    const int mav = (ml + mu) / 2;
    if (x < (float)kIq4nlValues[mav]) mu = mav; else ml = mav;
  }
  return (x - (float)kIq4nlValues[mu - 1] < (float)kIq4nlValues[mu] - x) ? (uint32_t)(mu - 1) : (uint32_t)mu;
}

__global__ __launch_bounds__(256) void quant_iq4nl_kernel(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                          int64_t nb, int32_t* __restrict__ src_block) {
  const int64_t ib = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (ib >= nb) return;
  const float* xb = x + ib * 32;
  float amax = 0.0f, max = 0.0f;
  for (int j = 0; j < 32; j++) {
    const float a = fabsf(xb[j]);
    if (a > amax) { amax = a; max = xb[j]; }
  }
  uint8_t* o = out + ib * 18;
  if (amax < 1e-15f) {
    o[0] = 0;
    o[1] = 0;
    src_block[ib] = -1;  // codes come from the last earlier non-zero block
    return;
  }
  src_block[ib] = (int32_t)ib;
  float d = max / (float)kIq4nlValues[0];
  const float id = 1.0f / d;
  float sumqx = 0.0f, sumq2 = 0.0f;
  uint8_t lv[32];
  for (int j = 0; j < 32; j++) {
    const uint32_t level = iq4_best_index(id * xb[j]);
    lv[j] = (uint8_t)level;
    const float q = (float)kIq4nlValues[level];
    const float w = xb[j] * xb[j];
    sumqx += w * q * xb[j];
    sumq2 += w * q * q;
  }
  d = sumq2 > 0.0f ? sumqx / sumq2 : 0.0f;
  const uint16_t dh = f2h(d);
  o[0] = (uint8_t)(dh & 0xFF);
  o[1] = (uint8_t)(dh >> 8);
  for (int j = 0; j < 16; j++) o[2 + j] = (uint8_t)(lv[j] | (lv[16 + j] << 4));
}

// One workgroup: running "last non-zero block" over all blocks, in chunks of
// 1024 with an inclusive max-scan per chunk.
__global__ __launch_bounds__(1024) void iq4nl_carry_kernel(uint8_t* __restrict__ out, int64_t nb,
                                                           const int32_t* __restrict__ src_block) {
  __shared__ int32_t s[1024];
  __shared__ int32_t carry;
  if (threadIdx.x == 0) carry = -1;
  __syncthreads();
  for (int64_t base = 0; base < nb; base += 1024) {
    const int64_t i = base + threadIdx.x;
    const int32_t mine = i < nb ? src_block[i] : -1;
    s[threadIdx.x] = mine;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int32_t v = threadIdx.x >= (unsigned)off ? s[threadIdx.x - off] : -1;
      __syncthreads();
      if (v > s[threadIdx.x]) s[threadIdx.x] = v;
      __syncthreads();
    }
    const int32_t c = carry;
    const int32_t last = s[threadIdx.x] > c ? s[threadIdx.x] : c;
    if (i < nb && mine < 0) {
      // a zero block: its codes are those of block `last`, or zero when none
      for (int j = 0; j < 16; j++) out[i * 18 + 2 + j] = last >= 0 ? out[(int64_t)last * 18 + 2 + j] : 0;
    }
    __syncthreads();
    if (threadIdx.x == 1023) carry = last;
    __syncthreads();
  }
}

size_t weight_quantize_scratch_bytes(int type, int64_t nelem) {
  return type == T_IQ4_NL ? (size_t)(nelem / 32) * 4 : 0;
}

hipError_t launch_weight_quantize(int type, const float* x, void* w, int64_t nelem, void* scratch, hipStream_t st) {
  switch (type) {
    case T_Q8_0: {
      const int64_t threads = (nelem / 32) * 8;
      const dim3 grid((unsigned)((threads + 255) / 256));
      if ((uintptr_t)x % 16 == 0)
        q8_0_kernel<true, true><<<grid, 256, 0, st>>>(x, nelem, nelem, 1, nullptr, nullptr, nullptr, (uint8_t*)w);
      else
        q8_0_kernel<false, true><<<grid, 256, 0, st>>>(x, nelem, nelem, 1, nullptr, nullptr, nullptr, (uint8_t*)w);
      break;
    }
    case T_Q4_K: {
      const int64_t nb = nelem / 256;
      quant_q4k_kernel<<<dim3((unsigned)((nb + 255) / 256)), 256, 0, st>>>(x, (uint8_t*)w, nb);
      break;
    }
    case T_Q6_K: {
      const int64_t nb = nelem / 256;
      quant_q6k_kernel<<<dim3((unsigned)((nb + 127) / 128)), 128, 0, st>>>(x, (uint8_t*)w, nb);
      break;
    }
    case T_MXFP4: {
      const int64_t nb = nelem / 32;
      quant_mxfp4_kernel<<<dim3((unsigned)((nb + 255) / 256)), 256, 0, st>>>(x, (uint8_t*)w, nb);
      break;
    }
    case T_IQ4_NL: {
      const int64_t nb = nelem / 32;
      quant_iq4nl_kernel<<<dim3((unsigned)((nb + 255) / 256)), 256, 0, st>>>(x, (uint8_t*)w, nb, (int32_t*)scratch);
      iq4nl_carry_kernel<<<1, 1024, 0, st>>>((uint8_t*)w, nb, (const int32_t*)scratch);
      break;
    }
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ===========================================================================
// dequantize (to_float), f32 or f16 out: one thread per 32 values.
// f16 output is f16(the f32 value) (dequantize_f16 == f16(dequantize)).
// ===========================================================================
template <typename OutT>
__device__ __forceinline__ void put(OutT* o, int64_t i, float v);
template <>
__device__ __forceinline__ void put<float>(float* o, int64_t i, float v) { o[i] = v; }
template <>
__device__ __forceinline__ void put<uint16_t>(uint16_t* o, int64_t i, float v) { o[i] = f2h(v); }

// The 32 values of group g (of 32 consecutive values) of a weight in GGUF
// blocks of `type`, to_float's arithmetic.
__device__ __forceinline__ void deq_group(int type, const uint8_t* __restrict__ w, int64_t g, float (&v)[32]) {
  switch (type) {
    case T_Q8_0: {
      const uint8_t* b = w + g * 34;
      const float d = h2f((uint16_t)(b[0] | (b[1] << 8)));
#pragma unroll
      for (int j = 0; j < 32; j++) v[j] = (float)(int8_t)b[2 + j] * d;
      break;
    }
    case T_MXFP4: {
      const uint8_t* b = w + g * 17;
      const float d = e8m0_half(b[0]);
#pragma unroll
      for (int j = 0; j < 16; j++) {
        v[j] = (float)kMxfp4Values[b[1 + j] & 0xF] * d;
        v[j + 16] = (float)kMxfp4Values[b[1 + j] >> 4] * d;
      }
      break;
    }
    case T_IQ4_NL: {
      const uint8_t* b = w + g * 18;
      const float d = h2f((uint16_t)(b[0] | (b[1] << 8)));
#pragma unroll
      for (int j = 0; j < 16; j++) {
        v[j] = d * (float)kIq4nlValues[b[2 + j] & 0xF];
        v[j + 16] = d * (float)kIq4nlValues[b[2 + j] >> 4];
      }
      break;
    }
    case T_Q4_K: {
      const int64_t sb = g >> 3;
      const int sub = (int)(g & 7);
      const uint8_t* b = w + sb * 144;
      const float d = h2f(*(const uint16_t*)b), mn = h2f(*(const uint16_t*)(b + 2));
      int sc, m;
      scale_min_k4(sub, b + 4, sc, m);
      const float d1 = d * (float)sc, m1 = mn * (float)m;
      const uint8_t* q = b + 16 + 32 * (sub >> 1);
      const int shift = (sub & 1) ? 4 : 0;
#pragma unroll
      for (int l = 0; l < 32; l++) v[l] = d1 * (float)((q[l] >> shift) & 0xF) - m1;
      break;
    }
    case T_Q6_K: {
      // group g: super-block sb, half h (0/1), quarter t (0..3) -> values 128h + 32t + l
      const int64_t sb = g >> 3;
      const int h = (int)((g >> 2) & 1), t = (int)(g & 3);
      const uint8_t* b = w + sb * 210;
      const float d = h2f((uint16_t)(b[208] | (b[209] << 8)));
      const int8_t* sc = (const int8_t*)(b + 192) + 8 * h;
      const uint8_t* ql = b + 64 * h;
      const uint8_t* qh = b + 128 + 32 * h;
#pragma unroll
      for (int l = 0; l < 32; l++) {
        const int lo = (t & 1) ? ql[l + 32] : ql[l];
        const int nib = (t & 2) ? (lo >> 4) : (lo & 0xF);
        const int q = (int)(int8_t)((nib | (((qh[l] >> (2 * t)) & 3) << 4)) - 32);
        v[l] = d * (float)sc[l / 16 + 2 * t] * (float)q;
      }
      break;
    }
    default:
#pragma unroll
      for (int l = 0; l < 32; l++) v[l] = 0.0f;
      break;
  }
}

template <typename OutT>
__global__ __launch_bounds__(256) void dequant_kernel(int type, const uint8_t* __restrict__ w, OutT* __restrict__ y,
                                                      int64_t ngroups) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;  // group of 32 outputs
  if (g >= ngroups) return;
  float v[32];
  deq_group(type, w, g, v);
#pragma unroll
  for (int j = 0; j < 32; j++) put(y, g * 32 + j, v[j]);
}

// The dequantize-then-multiply path the reference takes under set_force_dmmv
// (dequantize_mul_mat_vec and the dequantize + f32 matmul of
// quantized/cuda.rs:1653-1745): each weight value is dequantized as to_float
// does, multiplied by the f32 activation and summed in f32, with no
// activation quantization. A wave per weight row, lane L taking groups
// L, L + 64, ... of 32 values; up to kDmmvRows activation rows a launch.
constexpr int kDmmvRows = 8;

__global__ __launch_bounds__(256) void dmmv_kernel(int type, const uint8_t* __restrict__ w, int64_t n, int64_t k,
                                                   int64_t rowbytes, const float* __restrict__ x, int64_t xstride,
                                                   int nr, float* __restrict__ dst, int64_t ldd) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;  // whole waves
  const uint8_t* wr = w + row * rowbytes;
  const int64_t groups = k / 32;
  float acc[kDmmvRows];
#pragma unroll
  for (int r = 0; r < kDmmvRows; r++) acc[r] = 0.0f;
  for (int64_t g = lane; g < groups; g += 64) {
    float v[32];
    deq_group(type, wr, g, v);
#pragma unroll
    for (int r = 0; r < kDmmvRows; r++) {
      if (r >= nr) break;
      const float* xp = x + r * xstride + g * 32;
#pragma unroll
      for (int l = 0; l < 32; l++) acc[r] = __fmaf_rn(v[l], xp[l], acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < kDmmvRows; r++) {
    if (r >= nr) break;
    const float sum = wave_sum(acc[r]);
    if (lane == 0) dst[r * ldd + row] = sum;
  }
}

hipError_t launch_dmmv(int type, const void* w, int64_t n, int64_t k, const float* x, int64_t xstride, int64_t rows,
                       float* dst, int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  int64_t rowbytes;
  switch (type) {
    case T_Q8_0: rowbytes = k / 32 * 34; break;
    case T_IQ4_NL: rowbytes = k / 32 * 18; break;
    case T_MXFP4: rowbytes = k / 32 * 17; break;
    case T_Q4_K: rowbytes = k / 256 * 144; break;
    case T_Q6_K: rowbytes = k / 256 * 210; break;
    default: return hipErrorInvalidValue;
  }
  const dim3 grid((unsigned)((n + 3) / 4));
  for (int64_t r0 = 0; r0 < rows; r0 += kDmmvRows) {
    const int nr = (int)(rows - r0 < kDmmvRows ? rows - r0 : kDmmvRows);
    dmmv_kernel<<<grid, 256, 0, st>>>(type, (const uint8_t*)w, n, k, rowbytes, x + r0 * xstride, xstride, nr,
                                      dst + r0 * ldd, ldd);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_dequantize(int type, const void* w, void* out, int out_f16, int64_t nelem, hipStream_t st) {
  const int64_t groups = nelem / 32;
  const dim3 grid((unsigned)((groups + 255) / 256));
  if (out_f16)
    dequant_kernel<uint16_t><<<grid, 256, 0, st>>>(type, (const uint8_t*)w, (uint16_t*)out, groups);
  else
    dequant_kernel<float><<<grid, 256, 0, st>>>(type, (const uint8_t*)w, (float*)out, groups);
  return hipGetLastError();
}

// ===========================================================================
// Synthetic N(mean, std) data: splitmix64 counters -> Box-Muller in double.
// Element 2p and 2p+1 come from the pair of 53-bit uniforms drawn at
// counters seed + 2p and seed + 2p + 1.
// ===========================================================================
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void fill_normal_kernel(float* __restrict__ out, int64_t n, uint64_t seed, float mean,
                                                          float std) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (2 * p >= n) return;
  const double u1 = 1.0 - (double)(splitmix64(seed + 2 * (uint64_t)p) >> 11) * 0x1.0p-53;  // (0, 1]
  const double u2 = (double)(splitmix64(seed + 2 * (uint64_t)p + 1) >> 11) * 0x1.0p-53;
  const double r = sqrt(-2.0 * log(u1));
  const double a = 6.283185307179586 * u2;
  out[2 * p] = (float)((double)mean + (double)std * r * cos(a));
  if (2 * p + 1 < n) out[2 * p + 1] = (float)((double)mean + (double)std * r * sin(a));
}

hipError_t launch_fill_normal(float* out, int64_t n, uint64_t seed, float mean, float std, hipStream_t st) {
  const int64_t pairs = (n + 1) / 2;
  fill_normal_kernel<<<dim3((unsigned)((pairs + 255) / 256)), 256, 0, st>>>(out, n, seed, mean, std);
  return hipGetLastError();
}

}  // namespace qmm
