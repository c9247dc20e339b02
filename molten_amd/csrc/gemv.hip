// gemv.hip -- decode GEMVs over MLX affine Q4/Q6 weights for gfx950.
//
// Layout of the work: one wave64 owns R consecutive rows at a time and one
// 32-code chunk per lane (a K=2048 Q4 row is 64 lanes x 16 B, one coalesced
// dwordx4 per lane; a Q6 row is 64 lanes x 24 B).  Codes are dequantized in
// registers, products accumulate in f32 with fma in the chunk order (see
// mh_device.hpp), and the row value is the wave's xor-butterfly.  No MFMA:
// the path is HBM-bound at batch 1.  Waves loop over row groups with the next
// group's loads issued before the current group's arithmetic.
//
// Replaces lfm.metal:100-297 (GEMV_Q4_BODY, lfm_gemv_q4_bf16[_k*],
// lfm_gemv_q6_bf16[_x4]) and :1113-1386 (argmax, head argmax, token tail).
#include "mh_device.hpp"
#include "mh_host.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / mh::kWave;
constexpr int kXPitch = 36;  // LDS floats per staged x chunk (32 + 4: no bank conflicts)

struct GemvArgs {
    const uint32_t* codes;
    const uint16_t* scales;
    const uint16_t* biases;
    const uint16_t* x;        // bf16 [batch, k]
    uint16_t* y;              // bf16 [batch, n] or null
    unsigned long long* best; // [batch] keys, or the finisher scratch
    const void* done;         // non-null: finisher mode (best is the scratch)
    uint32_t* ids;            // [batch] tokens written by the finisher
    uint32_t n, k, gs, row_words, groups;
};

template <int BITS>
__device__ __forceinline__ void load_row_chunk(const GemvArgs& a, uint32_t row, uint32_t c,
                                               mh::Chunk<BITS>& ch, float& s, float& b) {
    ch.load(a.codes + static_cast<size_t>(row) * a.row_words + static_cast<size_t>(c) * BITS);
    const uint32_t g = (32u * c) / a.gs;
    s = mh::bf16_to_f32(a.scales[static_cast<size_t>(row) * a.groups + g]);
    b = mh::bf16_to_f32(a.biases[static_cast<size_t>(row) * a.groups + g]);
}

// Per-wave argmax state folded into the workgroup, then into the keys.
// bv/bi are wave-uniform.  Cross-workgroup traffic is atomic only: an
// atomic's returned value is consumed before the workgroup signals, so it has
// been performed at the coherence point and no cache write-back is needed.
//
// Without a finisher (a.done == null: the reference's gemv_head_argmax) every
// workgroup folds its key into best[b].  With the finisher, contention is a
// two-level tree: workgroup w folds into group key (w % G), the last
// workgroup of each group folds that into the final key, and the last group
// writes the token ids and re-zeroes the scratch (layout in molten_hip.h:
// group keys [G][B] | final keys [B] | group counters [G] | top counter).
constexpr uint32_t kArgGroups = MH_ARGMAX_GROUPS;

__device__ __forceinline__ unsigned long long amax(unsigned long long* p, unsigned long long v) {
    return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long axchg(unsigned long long* p, unsigned long long v) {
    return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long aadd(unsigned long long* p, unsigned long long v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int B>
__device__ void fold_argmax(const GemvArgs& a, const float (&bv)[B], const uint32_t (&bi)[B],
                            int lane, int wave) {
    __shared__ float sv[kWaves][B];
    __shared__ uint32_t si[kWaves][B];
    __shared__ uint32_t flag;
    __shared__ unsigned long long sink;
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            sv[wave][b] = bv[b];
            si[wave][b] = bi[b];
        }
    }
    __syncthreads();
    unsigned long long key = 0;
    if (threadIdx.x < B) {
        const int b = threadIdx.x;
        float v = sv[0][b];
        uint32_t i = si[0][b];
        for (int w = 1; w < kWaves; ++w) {
            mh::argmax_merge(v, i, sv[w][b], si[w][b]);
        }
        key = mh::argmax_key(v, i);
    }
    if (a.done == nullptr) {
        if (threadIdx.x < B) {
            amax(a.best + threadIdx.x, key);
        }
        return;
    }
    const uint32_t groups = min(gridDim.x, kArgGroups);
    const uint32_t g = blockIdx.x % groups;
    const uint32_t members = (gridDim.x - g + groups - 1) / groups;
    unsigned long long* gkeys = a.best;                      // [G][B]
    unsigned long long* fkeys = a.best + kArgGroups * B;     // [B]
    unsigned long long* gcnt = fkeys + B;                    // [G]
    unsigned long long* top = gcnt + kArgGroups;             // [1]
    if (threadIdx.x < B) {
        sink = amax(gkeys + g * B + threadIdx.x, key);  // performed before the barrier
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        flag = aadd(gcnt + g, 1ull) == members - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!flag) {
        return;
    }
    if (threadIdx.x < B) {
        const unsigned long long k = axchg(gkeys + g * B + threadIdx.x, 0ull);
        sink = amax(fkeys + threadIdx.x, k);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        axchg(gcnt + g, 0ull);
        flag = aadd(top, 1ull) == groups - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!flag) {
        return;
    }
    if (threadIdx.x < B) {
        const unsigned long long k = axchg(fkeys + threadIdx.x, 0ull);
        a.ids[threadIdx.x] = ~static_cast<uint32_t>(k & 0xffffffffull);
    }
    if (threadIdx.x == 0) {
        axchg(top, 0ull);
    }
}

// Row values (wave-uniform) of one row group: store and argmax.
template <int B, int R>
__device__ __forceinline__ void emit_rows(const GemvArgs& a, uint32_t rg, const float (&v)[R][B],
                                          float (&bv)[B], uint32_t (&bi)[B], int lane) {
    const uint32_t N = a.n;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        uint16_t mine = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint16_t vb = mh::f32_to_bf16(v[r][b]);
            const uint32_t row = rg * R + r;
            if (lane == r) {
                mine = vb;
            }
            if (a.best != nullptr && row < N) {
                mh::argmax_merge(bv[b], bi[b], mh::bf16_to_f32(vb), row);
            }
        }
        const uint32_t my_row = rg * R + lane;
        if (a.y != nullptr && lane < R && my_row < N) {
            a.y[static_cast<size_t>(b) * N + my_row] = mine;
        }
    }
}

// Batch 1, K <= 2048: each lane owns chunk `lane` of every row, with its x in
// registers for the whole kernel.  Waves are persistent over row groups and
// keep the next group's loads in flight during the current group's math.
// Row addresses are wave-uniform (scalar base + the lane's fixed offset), so
// the loads cost no vector ALU work.
template <int BITS, int R>
__global__ __launch_bounds__(kThreads) void k_gemv_b1(GemvArgs a) {
    const int lane = threadIdx.x & (mh::kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / mh::kWave);
    const uint32_t C = a.k / 32u;
    const uint32_t N = a.n;
    const bool live = lane < static_cast<int>(C);
    const uint32_t c = live ? lane : 0u;

    float xr[32];
    float xs;
    mh::load_x_chunk<BITS>(a.x + 32u * c, xr, xs);

    // lane-invariant byte offsets; row bases are scalar
    const uint32_t code_off = c * BITS * 4u;
    const uint32_t sb_off = ((32u * c) / a.gs) * 2u;
    const size_t row_bytes = static_cast<size_t>(a.row_words) * 4u;
    const size_t sb_row_bytes = static_cast<size_t>(a.groups) * 2u;
    const char* codes = reinterpret_cast<const char*>(a.codes);
    const char* scales = reinterpret_cast<const char*>(a.scales);
    const char* biases = reinterpret_cast<const char*>(a.biases);

    float bv[1] = {-__builtin_inff()};
    uint32_t bi[1] = {0u};
    const uint32_t n_rg = (N + R - 1) / R;
    const uint32_t stride = gridDim.x * kWaves;
    uint32_t rg = blockIdx.x * kWaves + wave;

    mh::Chunk<BITS> cur[R];
    float cs[R], cb[R];
    auto load_group = [&](uint32_t g, mh::Chunk<BITS>(&ch)[R], float(&s)[R], float(&b)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = min(g * R + r, N - 1);
            ch[r].load(mh::uniform_ptr(codes + row * row_bytes), code_off);
            s[r] = mh::bf16_to_f32(mh::gload<uint16_t>(mh::uniform_ptr(scales + row * sb_row_bytes), sb_off));
            b[r] = mh::bf16_to_f32(mh::gload<uint16_t>(mh::uniform_ptr(biases + row * sb_row_bytes), sb_off));
        }
    };
    if (rg < n_rg) {
        load_group(rg, cur, cs, cb);
    }
    while (rg < n_rg) {
        const uint32_t next = rg + stride;
        mh::Chunk<BITS> nxt[R];
        float ns[R], nb[R];
        if (next < n_rg) {
            load_group(next, nxt, ns, nb);
        }
        float v[R][1];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float p = cur[r].dot(xr);
            const float h = __builtin_fmaf(cs[r], p, cb[r] * xs);
            v[r][0] = mh::lane63(mh::wave_sum_lane63(live ? 0.0f + h : 0.0f));
        }
        emit_rows<1, R>(a, rg, v, bv, bi, lane);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            cur[r] = nxt[r];
            cs[r] = ns[r];
            cb[r] = nb[r];
        }
        rg = next;
    }
    if (a.best != nullptr) {
        fold_argmax<1>(a, bv, bi, lane, wave);
    }
}

// General form: any K, batch 1..8.  x is staged in LDS, one padded 32-float
// slot per (batch, chunk); lanes walk chunks c = lane, lane + 64, ...
template <int BITS, int B, int R>
__global__ __launch_bounds__(kThreads) void k_gemv_staged(GemvArgs a) {
    extern __shared__ float lds[];
    const int lane = threadIdx.x & (mh::kWave - 1);
    const int wave = threadIdx.x / mh::kWave;
    const uint32_t C = a.k / 32u;
    const uint32_t N = a.n;
    float* xl = lds;                                          // [B*C][kXPitch]
    float* xsl = lds + static_cast<size_t>(B) * C * kXPitch;  // [B*C]

    for (uint32_t t = threadIdx.x; t < B * C; t += kThreads) {
        const uint32_t b = t / C, c = t % C;
        float xc[32], s;
        mh::load_x_chunk<BITS>(a.x + static_cast<size_t>(b) * a.k + 32u * c, xc, s);
        float4* dst = reinterpret_cast<float4*>(xl + static_cast<size_t>(t) * kXPitch);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            dst[q] = make_float4(xc[4 * q], xc[4 * q + 1], xc[4 * q + 2], xc[4 * q + 3]);
        }
        xsl[t] = s;
    }
    __syncthreads();

    float bv[B];
    uint32_t bi[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        bv[b] = -__builtin_inff();
        bi[b] = 0u;
    }
    const uint32_t n_rg = (N + R - 1) / R;
    const uint32_t stride = gridDim.x * kWaves;
    for (uint32_t rg = blockIdx.x * kWaves + wave; rg < n_rg; rg += stride) {
        float acc[R][B];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                acc[r][b] = 0.0f;
            }
        }
        for (uint32_t c = lane; c < C; c += mh::kWave) {
            mh::Chunk<BITS> ch[R];
            float s[R], bb[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t row = min(rg * R + r, N - 1);
                load_row_chunk<BITS>(a, row, c, ch[r], s[r], bb[r]);
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                float xc[32];
                const float4* src =
                    reinterpret_cast<const float4*>(xl + (static_cast<size_t>(b) * C + c) * kXPitch);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 v = src[q];
                    xc[4 * q] = v.x;
                    xc[4 * q + 1] = v.y;
                    xc[4 * q + 2] = v.z;
                    xc[4 * q + 3] = v.w;
                }
                const float xs = xsl[static_cast<size_t>(b) * C + c];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float p = ch[r].dot(xc);
                    acc[r][b] = acc[r][b] + __builtin_fmaf(s[r], p, bb[r] * xs);
                }
            }
        }
        float v[R][B];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                v[r][b] = mh::lane63(mh::wave_sum_lane63(acc[r][b]));
            }
        }
        emit_rows<B, R>(a, rg, v, bv, bi, lane);
    }
    if (a.best != nullptr) {
        fold_argmax<B>(a, bv, bi, lane, wave);
    }
}

constexpr int kWgPerCu = 4;

template <typename K>
int launch_grid(K kernel, const GemvArgs& a, uint32_t rows_per_wave, size_t lds, hipStream_t stream,
                const char* name) {
    const uint32_t n_rg = (a.n + rows_per_wave - 1) / rows_per_wave;
    const uint32_t want = (n_rg + kWaves - 1) / kWaves;
    const uint32_t cap = static_cast<uint32_t>(mh::cu_count()) * kWgPerCu;
    const uint32_t grid = want < cap ? want : cap;
    if (lds > 64u * 1024u) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(lds));
        if (e != hipSuccess) {
            return mh::hip_error(e, name);
        }
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), lds, stream, a);
    return mh::launch_status(name);
}

template <int BITS, int B, int R>
int launch_staged(const GemvArgs& a, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(B) * (a.k / 32u) * (kXPitch + 1) * sizeof(float);
    return launch_grid(k_gemv_staged<BITS, B, R>, a, R, lds, stream, "k_gemv_staged");
}

template <int BITS>
int dispatch_gemv(const GemvArgs& a, uint32_t batch, hipStream_t stream) {
    switch (batch) {
        case 1:
            if (a.k <= 2048u) {
                return launch_grid(k_gemv_b1<BITS, 4>, a, 4, 0, stream, "k_gemv_b1");
            }
            return launch_staged<BITS, 1, 4>(a, stream);
        case 2: return launch_staged<BITS, 2, 2>(a, stream);
        case 3: return launch_staged<BITS, 3, 2>(a, stream);
        case 4: return launch_staged<BITS, 4, 2>(a, stream);
        case 5: return launch_staged<BITS, 5, 2>(a, stream);
        case 6: return launch_staged<BITS, 6, 2>(a, stream);
        case 7: return launch_staged<BITS, 7, 2>(a, stream);
        case 8: return launch_staged<BITS, 8, 2>(a, stream);
        default: return mh::set_error(MH_ERR_UNSUPPORTED, "gemv: batch %u not in 1..8", batch);
    }
}

// Largest LDS request of the staged path: B * C * (kXPitch + 1) floats.
constexpr size_t kMaxLds = 160u * 1024u;

int gemv_common(const char* op, const mh_quant_weights* w, const uint16_t* x, uint16_t* y,
                uint64_t* best, bool finisher, uint32_t* ids, uint32_t batch,
                mh_stream_t stream) {
    MH_TRY(mh::check_quant(w, op));
    MH_ENSURE(x != nullptr, MH_ERR_INVALID, "%s: x is NULL", op);
    MH_ENSURE(batch >= 1 && batch <= 8, MH_ERR_UNSUPPORTED, "%s: batch %u not in 1..8", op, batch);
    MH_ENSURE(mh::aligned(x, 2) && (y == nullptr || mh::aligned(y, 2)), MH_ERR_ALIGN,
              "%s: x/y not 2-byte aligned", op);
    MH_ENSURE(best == nullptr || mh::aligned(best, 8), MH_ERR_ALIGN,
              "%s: argmax key not 8-byte aligned", op);
    MH_ENSURE(!finisher || (best != nullptr && ids != nullptr), MH_ERR_INVALID,
              "%s: the argmax finisher needs the scratch and ids", op);
    const uint32_t C = w->in_features / 32u;
    const bool xreg = batch == 1 && w->in_features <= 2048u;
    MH_ENSURE(xreg || static_cast<size_t>(batch) * C * (kXPitch + 1) * 4 <= kMaxLds,
              MH_ERR_UNSUPPORTED, "%s: batch %u x in_features %u exceeds the LDS staging", op,
              batch, w->in_features);
    GemvArgs a{};
    a.codes = w->codes;
    a.scales = w->scales;
    a.biases = w->biases;
    a.x = x;
    a.y = y;
    a.best = reinterpret_cast<unsigned long long*>(best);
    a.done = finisher ? static_cast<const void*>(best) : nullptr;
    a.ids = ids;
    a.n = w->out_features;
    a.k = w->in_features;
    a.gs = w->group_size;
    a.row_words = w->in_features * w->bits / 32u;
    a.groups = w->in_features / w->group_size;
    const hipStream_t s = mh::as_stream(stream);
    return w->bits == 4 ? dispatch_gemv<4>(a, batch, s) : dispatch_gemv<6>(a, batch, s);
}

// ------------------------------------------------------------- dequant ---

template <int BITS>
__global__ __launch_bounds__(256) void k_dequant(const uint32_t* codes, const uint16_t* scales,
                                                 const uint16_t* biases, uint16_t* out,
                                                 uint32_t n, uint32_t k, uint32_t gs) {
    const uint32_t C = k / 32u;
    const size_t total = static_cast<size_t>(n) * C;
    const uint32_t row_words = k * BITS / 32u;
    const uint32_t groups = k / gs;
    for (size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const uint32_t row = static_cast<uint32_t>(t / C);
        const uint32_t c = static_cast<uint32_t>(t % C);
        mh::Chunk<BITS> ch;
        ch.load(codes + static_cast<size_t>(row) * row_words + static_cast<size_t>(c) * BITS);
        const uint32_t g = 32u * c / gs;
        const float s = mh::bf16_to_f32(scales[static_cast<size_t>(row) * groups + g]);
        const float b = mh::bf16_to_f32(biases[static_cast<size_t>(row) * groups + g]);
        uint32_t packed[16];
#pragma unroll
        for (int i = 0; i < 32; i += 2) {
            uint32_t q0, q1;
            if constexpr (BITS == 4) {
                q0 = (ch.w[i >> 3] >> (4 * (i & 7))) & 15u;
                q1 = (ch.w[(i + 1) >> 3] >> (4 * ((i + 1) & 7))) & 15u;
            } else {
                const int b0 = 6 * i, b1 = 6 * (i + 1);
                q0 = ((b0 & 31) + 6 <= 32) ? (ch.w[b0 >> 5] >> (b0 & 31)) & 63u
                                           : __builtin_amdgcn_alignbit(ch.w[(b0 >> 5) + 1], ch.w[b0 >> 5], b0 & 31) & 63u;
                q1 = ((b1 & 31) + 6 <= 32) ? (ch.w[b1 >> 5] >> (b1 & 31)) & 63u
                                           : __builtin_amdgcn_alignbit(ch.w[(b1 >> 5) + 1], ch.w[b1 >> 5], b1 & 31) & 63u;
            }
            const uint16_t lo = mh::f32_to_bf16(__builtin_fmaf(s, static_cast<float>(q0), b));
            const uint16_t hi = mh::f32_to_bf16(__builtin_fmaf(s, static_cast<float>(q1), b));
            packed[i >> 1] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
        }
        uint4* dst = reinterpret_cast<uint4*>(out + static_cast<size_t>(row) * k + 32u * c);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            dst[q] = make_uint4(packed[4 * q], packed[4 * q + 1], packed[4 * q + 2], packed[4 * q + 3]);
        }
    }
}

int dequant_common(const char* op, const mh_quant_weights* w, uint16_t* out, mh_stream_t stream) {
    MH_TRY(mh::check_quant(w, op));
    MH_ENSURE(out != nullptr, MH_ERR_INVALID, "%s: out is NULL", op);
    MH_ENSURE(mh::aligned(out, 16), MH_ERR_ALIGN, "%s: out not 16-byte aligned", op);
    const size_t total = static_cast<size_t>(w->out_features) * (w->in_features / 32u);
    const size_t want = (total + 255) / 256;
    const size_t cap = static_cast<size_t>(mh::cu_count()) * 16;
    const unsigned grid = static_cast<unsigned>(want < cap ? want : cap);
    const hipStream_t s = mh::as_stream(stream);
    if (w->bits == 4) {
        hipLaunchKernelGGL(k_dequant<4>, dim3(grid), dim3(256), 0, s, w->codes, w->scales,
                           w->biases, out, w->out_features, w->in_features, w->group_size);
    } else {
        hipLaunchKernelGGL(k_dequant<6>, dim3(grid), dim3(256), 0, s, w->codes, w->scales,
                           w->biases, out, w->out_features, w->in_features, w->group_size);
    }
    return mh::launch_status(op);
}

// ----------------------------------------------------------- token tail ---

__global__ void k_token_tail(unsigned long long* best, uint32_t* out_tok, uint32_t batch) {
    const uint32_t b = threadIdx.x;
    if (b < batch) {
        const unsigned long long key = best[b];
        best[b] = 0ull;
        out_tok[b] = ~static_cast<uint32_t>(key & 0xffffffffull);
    }
}

// --------------------------------------------------- two-stage argmax ---

constexpr int kArgmaxGroups = 64;

struct ArgPair {
    float v;
    uint32_t i;
};

__device__ void block_argmax(float& bv, uint32_t& bi) {
    __shared__ float sv[256 / mh::kWave];
    __shared__ uint32_t si[256 / mh::kWave];
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        mh::argmax_merge(bv, bi, ov, oi);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < static_cast<int>(blockDim.x / mh::kWave); ++w) {
            mh::argmax_merge(bv, bi, sv[w], si[w]);
        }
    }
}

__global__ __launch_bounds__(256) void k_argmax_partial(const uint16_t* x, ArgPair* partials,
                                                        uint32_t n, uint32_t chunk) {
    float bv = -__builtin_inff();
    uint32_t bi = 0;
    const uint32_t begin = blockIdx.x * chunk;
    const uint32_t end = min(begin + chunk, n);
    for (uint32_t i = begin + threadIdx.x; i < end; i += blockDim.x) {
        mh::argmax_merge(bv, bi, mh::bf16_to_f32(x[i]), i);
    }
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
        partials[blockIdx.x].v = bv;
        partials[blockIdx.x].i = bi;
    }
}

__global__ __launch_bounds__(256) void k_argmax_final(const ArgPair* partials, uint32_t* out,
                                                      uint32_t groups) {
    float bv = -__builtin_inff();
    uint32_t bi = 0;
    for (uint32_t g = threadIdx.x; g < groups; g += blockDim.x) {
        mh::argmax_merge(bv, bi, partials[g].v, partials[g].i);
    }
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
        out[0] = bi;
    }
}

}  // namespace

extern "C" {

int mh_gemv_quant(const mh_quant_weights* w, const uint16_t* x, uint16_t* y, uint32_t batch,
                  mh_stream_t stream) {
    MH_ENSURE(y != nullptr, MH_ERR_INVALID, "mh_gemv_quant: y is NULL");
    return gemv_common("mh_gemv_quant", w, x, y, nullptr, false, nullptr, batch, stream);
}

int mh_gemv_head_argmax(const mh_quant_weights* w, const uint16_t* x, uint64_t* best,
                        uint32_t batch, mh_stream_t stream) {
    MH_ENSURE(best != nullptr, MH_ERR_INVALID, "mh_gemv_head_argmax: best is NULL");
    return gemv_common("mh_gemv_head_argmax", w, x, nullptr, best, false, nullptr, batch,
                       stream);
}

int mh_gemv_quant_argmax(const mh_quant_weights* w, const uint16_t* x, uint16_t* y,
                         uint64_t* scratch, uint32_t* ids, uint32_t batch, mh_stream_t stream) {
    MH_ENSURE(scratch != nullptr && ids != nullptr, MH_ERR_INVALID,
              "mh_gemv_quant_argmax: scratch/ids is NULL");
    return gemv_common("mh_gemv_quant_argmax", w, x, y, scratch, true, ids, batch, stream);
}

int mh_token_tail(uint64_t* best, uint32_t* out_tok, uint32_t batch, mh_stream_t stream) {
    MH_ENSURE(best != nullptr && out_tok != nullptr, MH_ERR_INVALID,
              "mh_token_tail: best/out_tok is NULL");
    MH_ENSURE(mh::aligned(best, 8), MH_ERR_ALIGN, "mh_token_tail: key not 8-byte aligned");
    MH_ENSURE(batch >= 1 && batch <= 64, MH_ERR_INVALID, "mh_token_tail: batch %u not in 1..64",
              batch);
    hipLaunchKernelGGL(k_token_tail, dim3(1), dim3(64), 0, mh::as_stream(stream),
                       reinterpret_cast<unsigned long long*>(best), out_tok, batch);
    return mh::launch_status("mh_token_tail");
}

int mh_argmax_bf16(const uint16_t* x, uint32_t n, void* partials, uint32_t* out,
                   mh_stream_t stream) {
    MH_ENSURE(x && partials && out, MH_ERR_INVALID, "mh_argmax_bf16: NULL argument");
    MH_ENSURE(n > 0, MH_ERR_INVALID, "mh_argmax_bf16: empty input");
    MH_ENSURE(mh::aligned(partials, 8), MH_ERR_ALIGN, "mh_argmax_bf16: partials not 8-byte aligned");
    const uint32_t chunk = (n + kArgmaxGroups - 1) / kArgmaxGroups;
    const hipStream_t s = mh::as_stream(stream);
    hipLaunchKernelGGL(k_argmax_partial, dim3(kArgmaxGroups), dim3(256), 0, s, x,
                       static_cast<ArgPair*>(partials), n, chunk);
    MH_TRY(mh::launch_status("k_argmax_partial"));
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s,
                       static_cast<const ArgPair*>(partials), out,
                       static_cast<uint32_t>(kArgmaxGroups));
    return mh::launch_status("k_argmax_final");
}

int mh_dequant_to_bf16(const mh_quant_weights* w, uint16_t* out, mh_stream_t stream) {
    return dequant_common("mh_dequant_to_bf16", w, out, stream);
}

int mh_dequant_q4_bf16_bulk(const mh_quant_weights* w, uint16_t* out, mh_stream_t stream) {
    MH_ENSURE(w != nullptr && w->bits == 4 && w->in_features % 128 == 0, MH_ERR_INVALID,
              "mh_dequant_q4_bf16_bulk: bulk dequant needs 4-bit weights with K %% 128 == 0");
    return dequant_common("mh_dequant_q4_bf16_bulk", w, out, stream);
}

}  // extern "C"
