// hq_gemv.hip - batch-1 packed-int4 x int8 GEMV for gfx950, with the
// per-token int8 activation quantization (and optionally the RMSNorm in
// front of it) fused into the prologue and the residual add, SwiGLU or
// argmax fused into the epilogue.
//
// Restates cpu_kernels/litespark_int4.cpp:22-76 (reference repository):
// acc[n] = sum_k W[n,k] * x[k] in int32, out[n] = ((float)acc * act) * s[n].
//
// Two kernel shapes share the prologue and the dot products:
//   * gemv_kernel: 256-thread blocks of RB rows (the gate_up GEMV with
//     SwiGLU, the LM head with argmax, persistent over its tiles);
//   * gemv_rr_kernel: one block per CU with an equal share of the rows, one
//     wave tile each (the reference-ABI entry points and the qkv, o and
//     down step GEMVs);
// and in both:
//   * a row is read by LPR lanes, each lane loading whole 16-byte chunks
//     (32 int4 values) with 128-bit loads, so the lanes of a row read
//     LPR*16 contiguous bytes of it per load;
//   * all weight loads of a lane are issued before the activation prologue,
//     so the HBM stream is in flight while the block quantizes x;
//   * the prologue writes x as int8 into LDS, de-interleaved per 8 columns
//     (4 even columns, then 4 odd) to match the nibble order of a weight
//     dword;
//   * nibbles are decoded in registers right before the dot products:
//     for a weight dword w, (w << 4) & 0xF0F0F0F0 holds 16*low nibbles and
//     w & 0xF0F0F0F0 holds 16*high nibbles as signed bytes, so two
//     v_dot4_i32_i8 give 16 * sum(w*x) exactly; the 8-lane xor reduction
//     and a shift by 4 give the int32 accumulator (|16*acc| < 2^31 for
//     K <= 9728*2 with |w| <= 7, |x| <= 127).
#include "hq_device.h"
#include "hq_int4.h"
#include "hq_internal.h"

namespace hq {

// Activation registers: element i = tid + 256*j of x (and gamma) is held
// by thread tid, which for PRO_RMSNORM is exactly the spec's 256-lane
// partial sum of squares.  Loads are unconditional (clamped index) so the
// compiler issues them back to back before any use.
template <int XJ, int PRO>
struct ActRegs {
    float x[XJ];
    float g[PRO == PRO_RMSNORM ? XJ : 1];
};

template <int XJ, int PRO>
__device__ __forceinline__ void load_activation(const GemvParams& p, ActRegs<XJ, PRO>& a)
{
    if constexpr (PRO != PRO_I8) {
        const int K = p.width;
#pragma unroll
        for (int j = 0; j < XJ; ++j) {
            const int i = min(int(threadIdx.x) + kBlock * j, K - 1);
            a.x[j] = p.xf[i];
            if constexpr (PRO == PRO_RMSNORM) a.g[j] = p.gamma[i];
        }
    }
}

// Activation prologue: fills xs (width bytes, de-interleaved int8) and
// returns the act scale.
template <int XJ, int PRO>
__device__ __forceinline__ float activation_prologue(const GemvParams& p, ActRegs<XJ, PRO>& a,
                                                     uint8_t* xs, float* red)
{
    const int tid = threadIdx.x;
    const int K = p.width;
    if constexpr (PRO == PRO_I8) {
        for (int i = tid; i < K; i += kBlock) xs[xq_offset(i)] = uint8_t(p.xq[i]);
        return p.act_scale;
    } else {
        if constexpr (PRO == PRO_RMSNORM) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < XJ; ++j)
                if (tid + kBlock * j < K) ss = __builtin_fmaf(a.x[j], a.x[j], ss);
            const float total = block_tree_sum256(ss, red);
            const float ms = total / float(K);
            const float r = __builtin_sqrtf(ms + p.eps);
#pragma unroll
            for (int j = 0; j < XJ; ++j) a.x[j] = (a.x[j] / r) * a.g[j];
        }
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < XJ; ++j)
            if (tid + kBlock * j < K) amax = fmaxf(amax, fabsf(a.x[j]));
        amax = block_max_nonneg(amax, red);
        amax = fmaxf(amax, 1e-5f);
        const float inv = 127.0f / amax;
        const bool write_q = p.q_out != nullptr && blockIdx.x == 0;
#pragma unroll
        for (int j = 0; j < XJ; ++j) {
            const int i = tid + kBlock * j;
            if (i < K) {
                const int8_t q = quant_i8(a.x[j], inv);
                xs[xq_offset(i)] = uint8_t(q);
                if (write_q) p.q_out[i] = q;
            }
        }
        const float act = amax / 127.0f;
        if (p.act_out != nullptr && blockIdx.x == 0 && tid == 0) *p.act_out = act;
        return act;
    }
}

// ---------------------------------------------------------------------------
// Kernel shape: a wave owns whole rows.  LPR lanes (8, 16, 32 or 64) read one
// row, RPW = 64 / LPR rows per wave, RB = 4 * RPW rows per 256-thread block
// (a "tile").  Lane l of a row loads chunks l, l + LPR, ... (16 bytes = 32
// int4 values each), so a row's lanes read LPR*16 contiguous bytes per load.
// Row sums leave the wave through DPP and readlane: no LDS and no barrier
// between the dot products and the epilogue.  With EPI_SWIGLU, RPW = 2 and
// a wave's rows are gate rows followed by the matching up rows.
template <int LPR, int EPI>
__device__ __forceinline__ int wave_row(const GemvParams& p, int tile, int wave, int r, bool& valid)
{
    constexpr int RPW = kWave / LPR;
    if constexpr (EPI == EPI_SWIGLU) {
        // the wave's rows 0..RPW/2-1 are gate rows, the next RPW/2 the
        // matching up rows
        constexpr int PPW = RPW / 2;
        static_assert(PPW >= 1, "SwiGLU tiles need at least two rows per wave");
        const int pair = (tile * 4 + wave) * PPW + (r % PPW);
        valid = pair < p.half_rows;
        return r < PPW ? pair : p.half_rows + pair;
    } else {
        const int row = (tile * 4 + wave) * RPW + r;
        valid = row < p.rows;
        return row;
    }
}

// The epilogue operands of this lane's row of a tile (lane r < RPW
// finishes row r of its wave): the row scale (SwiGLU: gate and up scales)
// and, for EPI_RESIDUAL, the residual value.  Loaded with the tile's
// weights, so the epilogue waits for no memory round trip of its own;
// clamped (unconditional) loads, a row past the matrix re-reads the last.
struct EpiOperands {
    float s0, s1, x;
};
template <int LPR, int EPI>
__device__ __forceinline__ EpiOperands load_epi(const GemvParams& p, int tile, int wave, int lane)
{
    EpiOperands e{0.0f, 0.0f, 0.0f};
    bool ok;
    const int r = wave_row<LPR, EPI>(p, tile, wave, lane % (kWave / LPR), ok);
    if constexpr (EPI == EPI_SWIGLU) {
        const int gr = min(r, p.half_rows - 1);
        e.s0 = p.ws[gr];
        e.s1 = p.ws[p.half_rows + gr];
    } else {
        const int rr = min(r, p.rows - 1);
        e.s0 = p.ws[rr];
        if constexpr (EPI == EPI_RESIDUAL) e.x = p.out[rr];
    }
    return e;
}

template <int MAXC, int LPR>
__device__ __forceinline__ void load_tile(const uint8_t* wrow, int li, int nchunks, uint4 (&wv)[MAXC])
{
    // unconditional (clamped) loads: no branch separates them, so the wait
    // counters stay exact; chunks past the row are skipped in the dot loop
#pragma unroll
    for (int j = 0; j < MAXC; ++j) wv[j] = load_w16(wrow + size_t(min(li + j * LPR, nchunks - 1)) * 16);
}

// Tiles: non-persistent launches give each block one tile (and walk wide
// rows in batches of MAXC chunks per lane); persistent launches (PERSIST)
// loop over tiles blockIdx.x + k*gridDim.x with the next tile's weights in
// flight during the current tile's dot products, and need
// width <= MAXC*LPR*32.
template <int LPR, int MAXC, int XJ, int PRO, int EPI, bool PERSIST>
__global__ __launch_bounds__(kBlock) void gemv_kernel(GemvParams p)
{
    constexpr int RPW = kWave / LPR;
    constexpr int RB = 4 * RPW;
    extern __shared__ __align__(16) uint8_t xs[];
    __shared__ float red[kBlock];
    __shared__ float bval[kBlock / kWave];
    __shared__ int bidx[kBlock / kWave];
    __shared__ int last_flag;

    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int rsel = lane / LPR;          // row of the wave this lane reads
    const int li = lane % LPR;            // lane within the row
    const int K = p.width;
    const int nchunks = K >> 5;
    const int ntiles = (EPI == EPI_SWIGLU) ? (p.half_rows + RB / 2 - 1) / (RB / 2)
                                           : (p.rows + RB - 1) / RB;

    // 1. activation loads, then the first tile's weight loads
    ActRegs<XJ, PRO> areg;
    load_activation<XJ, PRO>(p, areg);
    int tile = blockIdx.x;
    bool valid;
    int row = wave_row<LPR, EPI>(p, tile, wave, rsel, valid);
    const uint8_t* wrow = p.w + size_t(valid ? row : 0) * size_t(K >> 1);
    uint4 wv[MAXC];
    load_tile<MAXC, LPR>(wrow, li, nchunks, wv);
    EpiOperands eo = load_epi<LPR, EPI>(p, tile, wave, lane);
    // keep the scheduler from sinking the weight loads below the first use
    // of the activations: the HBM stream must start before any wait
    __builtin_amdgcn_sched_barrier(0);

    // 2. activations -> LDS (overlaps the weight stream: the barriers of the
    // prologue wait for LDS only, not for the weight loads in flight)
    const float act = activation_prologue<XJ, PRO>(p, areg, xs, red);
    lds_sync();

    float best_v = -__builtin_inff();   // EPI_ARGMAX: running best of this lane's rows
    int best_i = 0x7FFFFFFF;
    while (true) {
        // 3. prefetch the next tile (persistent), dot products of this one
        const int next = tile + int(gridDim.x);
        uint4 wn[PERSIST ? MAXC : 1];
        EpiOperands en{};
        if constexpr (PERSIST) {
            if (next < ntiles) {
                bool nvalid;
                const int nrow = wave_row<LPR, EPI>(p, next, wave, rsel, nvalid);
                load_tile<MAXC, LPR>(p.w + size_t(nvalid ? nrow : 0) * size_t(K >> 1), li, nchunks, wn);
                en = load_epi<LPR, EPI>(p, next, wave, lane);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        int a0 = 0, a1 = 0, a2 = 0, a3 = 0;
#pragma unroll
        for (int j = 0; j < MAXC; ++j) {
            const int c = li + j * LPR;
            if (c < nchunks) {
                if (j & 1) dot_chunk(wv[j], xs + c * 32, a2, a3);
                else dot_chunk(wv[j], xs + c * 32, a0, a1);
            }
        }
        if constexpr (!PERSIST) {
            for (int base = MAXC * LPR; base < nchunks; base += MAXC * LPR) {
#pragma unroll
                for (int j = 0; j < MAXC; ++j)
                    wv[j] = load_w16(wrow + size_t(min(base + li + j * LPR, nchunks - 1)) * 16);
#pragma unroll
                for (int j = 0; j < MAXC; ++j) {
                    const int c = base + li + j * LPR;
                    if (c < nchunks) {
                        if (j & 1) dot_chunk(wv[j], xs + c * 32, a2, a3);
                        else dot_chunk(wv[j], xs + c * 32, a0, a1);
                    }
                }
            }
        }
        const int part = (a0 + a1) + (a2 + a3);

        // 4. epilogue of this tile: lane r < RPW finishes row r of the wave
        int acc = 0;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int t = row_isum<LPR>(part, r) >> 4;
            if (lane == r) acc = t;
        }
        if constexpr (EPI == EPI_SWIGLU) {
            constexpr int PPW = RPW / 2;
            int acc_up = 0;
#pragma unroll
            for (int r = 0; r < PPW; ++r) {
                const int t = row_isum<LPR>(part, r + PPW) >> 4;
                if (lane == r) acc_up = t;
            }
            if (lane < PPW) {
                bool ok;
                const int gr = wave_row<LPR, EPI>(p, tile, wave, lane, ok);
                if (ok) {
                    const int ur = p.half_rows + gr;
                    const float g = (float(acc) * act) * eo.s0;
                    const float u = (float(acc_up) * act) * eo.s1;
                    if (p.acc_out) { p.acc_out[gr] = acc; p.acc_out[ur] = acc_up; }
                    if (p.out_aux) { p.out_aux[gr] = g; p.out_aux[ur] = u; }
                    const float t = 1.0f + spec_expf(-g);
                    p.out[gr] = (g / t) * u;
                }
            }
        } else if (lane < RPW) {
            bool ok;
            const int r = wave_row<LPR, EPI>(p, tile, wave, lane, ok);
            if (ok) {
                const float v = (float(acc) * act) * eo.s0;
                if (p.acc_out) p.acc_out[r] = acc;
                if constexpr (EPI == EPI_STORE) {
                    p.out[r] = v;
                } else if constexpr (EPI == EPI_RESIDUAL) {
                    if (p.out_aux) p.out_aux[r] = v;
                    p.out[r] = eo.x + v;
                } else {   // EPI_ARGMAX
                    p.out[r] = v;
                    if (argmax_better(v, r, best_v, best_i)) { best_v = v; best_i = r; }
                }
            }
        }
        if constexpr (!PERSIST) break;
        if (next >= ntiles) break;
#pragma unroll
        for (int j = 0; j < MAXC; ++j) wv[j] = wn[j];
        eo = en;
        tile = next;
    }

    if constexpr (EPI == EPI_ARGMAX) {
        // block best, then the last block to arrive reduces the per-block
        // partials (no waiting)
        float v = best_v;
        int idx = best_i;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(v, o, kWave);
            const int oi = __shfl_xor(idx, o, kWave);
            if (argmax_better(ov, oi, v, idx)) { v = ov; idx = oi; }
        }
        if (lane == 0) { bval[wave] = v; bidx[wave] = idx; }
        __syncthreads();
        if (tid == 0) {
#pragma unroll
            for (int w = 1; w < kBlock / kWave; ++w)
                if (argmax_better(bval[w], bidx[w], v, idx)) { v = bval[w]; idx = bidx[w]; }
            publish_f(p.part_val + blockIdx.x, v);
            publish_i(p.part_idx + blockIdx.x, idx);
            wait_all_memory();
            last_flag = last_block_ticket(p.counter, blockIdx.x, gridDim.x);
        }
        __syncthreads();
        if (last_flag) {
            v = -__builtin_inff();
            idx = 0x7FFFFFFF;
            for (int b = tid; b < int(gridDim.x); b += kBlock) {
                const float bv = read_f(p.part_val + b);
                const int bi = read_i(p.part_idx + b);
                if (argmax_better(bv, bi, v, idx)) { v = bv; idx = bi; }
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const float ov = __shfl_xor(v, o, kWave);
                const int oi = __shfl_xor(idx, o, kWave);
                if (argmax_better(ov, oi, v, idx)) { v = ov; idx = oi; }
            }
            __syncthreads();
            if (lane == 0) { bval[wave] = v; bidx[wave] = idx; }
            __syncthreads();
            if (tid == 0) {
#pragma unroll
                for (int w = 1; w < kBlock / kWave; ++w)
                    if (argmax_better(bval[w], bidx[w], v, idx)) { v = bval[w]; idx = bidx[w]; }
                *p.token = idx;
                *p.position = *p.position + 1;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Row-range GEMV: one block per CU.  The rows are cut into wave tiles of
// RPW = 64/LPR rows, and block b owns tiles [b*tpb, (b+1)*tpb) (tpb = the
// tiles per block, ceil(tiles / CUs)), one tile per wave, so every CU
// streams the same number of rows and no wave loads a row it does not
// finish.  Each lane holds its C chunks of the row in registers, issued
// before the activation prologue (wider rows walk further batches of C
// chunks after the first).  The prologue (quantization, or RMSNorm then
// quantization, with exactly gemv_kernel's arithmetic) runs on waves 0-3,
// element i on thread i % 256; the other waves only meet its barriers.

// Waves 0-3 load the activations (element tid + 256*j, clamped); the other
// waves load element 0 (one cache line), so every wave issues the same
// unconditional loads ahead of its weight loads.
template <int XJ, int PRO>
__device__ __forceinline__ void rr_load_activation(const GemvParams& p, ActRegs<XJ, PRO>& a)
{
    if constexpr (PRO != PRO_I8) {
        const int K = p.width;
        const int tid = int(threadIdx.x);
#pragma unroll
        for (int j = 0; j < XJ; ++j) {
            const int i = tid < kBlock ? min(tid + kBlock * j, K - 1) : 0;
            a.x[j] = p.xf[i];
            if constexpr (PRO == PRO_RMSNORM) a.g[j] = p.gamma[i];
        }
    }
}

template <int XJ, int PRO>
__device__ __forceinline__ float rr_prologue(const GemvParams& p, ActRegs<XJ, PRO>& a, uint8_t* xs, float* red)
{
    const int tid = int(threadIdx.x);
    const int K = p.width;
    if constexpr (PRO == PRO_I8) {
        for (int i = tid; i < K; i += int(blockDim.x)) xs[xq_offset(i)] = uint8_t(p.xq[i]);
        return p.act_scale;
    } else {
        const bool pro = tid < kBlock;
        if constexpr (PRO == PRO_RMSNORM) {
            // the spec's 256 strided partials and halving tree
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < XJ; ++j)
                if (pro && tid + kBlock * j < K) ss = __builtin_fmaf(a.x[j], a.x[j], ss);
            if (pro) red[tid] = ss;
            lds_sync();
            const int l = tid & (kWave - 1);
            const float total = wave_tree_sum64_all((red[l] + red[l + 128]) + (red[l + 64] + red[l + 192]));
            lds_sync();   // red is written again below
            const float r = __builtin_sqrtf(total / float(K) + p.eps);
#pragma unroll
            for (int j = 0; j < XJ; ++j) a.x[j] = (a.x[j] / r) * a.g[j];
        }
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < XJ; ++j)
            if (pro && tid + kBlock * j < K) amax = fmaxf(amax, fabsf(a.x[j]));
        amax = wave_max64_all(amax);
        if (pro && (tid & (kWave - 1)) == 0) red[tid / kWave] = amax;
        lds_sync();
        amax = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), 1e-5f);
        const float inv = 127.0f / amax;
        const bool write_q = p.q_out != nullptr && blockIdx.x == 0;
        if (pro) {
#pragma unroll
            for (int j = 0; j < XJ; ++j) {
                const int i = tid + kBlock * j;
                if (i < K) {
                    const int8_t q = quant_i8(a.x[j], inv);
                    xs[xq_offset(i)] = uint8_t(q);
                    if (write_q) p.q_out[i] = q;
                }
            }
        }
        const float act = amax / 127.0f;
        if (p.act_out != nullptr && blockIdx.x == 0 && tid == 0) *p.act_out = act;
        return act;
    }
}

template <int LPR, int C, int XJ, int PRO, int EPI>
__global__ __launch_bounds__(1024) void gemv_rr_kernel(GemvParams p, int tpb)
{
    static_assert(EPI == EPI_STORE || EPI == EPI_RESIDUAL, "row-range epilogues: store, residual");
    constexpr int RPW = kWave / LPR;
    extern __shared__ __align__(16) uint8_t xs[];
    __shared__ float red[kBlock];

    const int tid = int(threadIdx.x);
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int li = lane % LPR;
    const int K = p.width;
    const int nchunks = K >> 5;
    // this wave's tile: rows row0 .. row0+RPW-1 (the last tile of the
    // matrix may hold fewer: its missing rows re-read the matrix's last row)
    const int row0 = (int(blockIdx.x) * tpb + wave) * RPW;
    const int row = min(row0 + lane / LPR, p.rows - 1);

    // 1. activation loads, then the weights of the first C chunks of the
    // row, then the epilogue operands of the row lane r < RPW finishes.
    // The prologue waves issue their weight loads once the activations
    // have arrived: issued behind the block's weight loads, the activation
    // loads wait for them in the memory pipeline and the prologue ends
    // after the weights (K 2560 -> 9728 rows, 8 lanes per row: 5.69 -> 5.11 us
    // per call).
    ActRegs<XJ, PRO> areg;
    rr_load_activation<XJ, PRO>(p, areg);
    const uint8_t* wrow = p.w + size_t(row) * size_t(K >> 1);
    uint4 wv[C];
    // A prologue wave issues half its chunks ahead of its activation wait
    // (exact: vmcnt counts its loads in issue order), so more of the weight
    // stream starts with the launch: K 2560 -> 9728 rows 5.09 -> 4.97 us per
    // call, qkv 4.38 -> 4.33, down 7.43 -> 7.36; the 32-lane rows (o, K 4096)
    // issue none early (4.16 -> 4.69 us with half).
    constexpr int CE = LPR == 32 ? 0 : C / 2;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < CE; ++j) wv[j] = load_w16(wrow + size_t(min(li + j * LPR, nchunks - 1)) * 16);
    __builtin_amdgcn_sched_barrier(0);
    if (__builtin_amdgcn_readfirstlane(wave) < 4) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CE) : "memory");
#pragma unroll
    for (int j = CE; j < C; ++j) wv[j] = load_w16(wrow + size_t(min(li + j * LPR, nchunks - 1)) * 16);
    const int erow = min(row0 + lane % RPW, p.rows - 1);
    const float es = p.ws[erow];
    float ex = 0.0f;
    if constexpr (EPI == EPI_RESIDUAL) ex = p.out[erow];
    __builtin_amdgcn_sched_barrier(0);

    // 2. activations -> LDS while the weights stream
    const float act = rr_prologue<XJ, PRO>(p, areg, xs, red);
    lds_sync();

    // 3. dot products (rows wider than C*LPR chunks take more batches)
    int a0 = 0, a1 = 0, a2 = 0, a3 = 0;
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const int c = li + j * LPR;
        if (c < nchunks) {
            if (j & 1) dot_chunk(wv[j], xs + c * 32, a2, a3);
            else dot_chunk(wv[j], xs + c * 32, a0, a1);
        }
    }
    for (int base = C * LPR; base < nchunks; base += C * LPR) {
#pragma unroll
        for (int j = 0; j < C; ++j) wv[j] = load_w16(wrow + size_t(min(base + li + j * LPR, nchunks - 1)) * 16);
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const int c = base + li + j * LPR;
            if (c < nchunks) {
                if (j & 1) dot_chunk(wv[j], xs + c * 32, a2, a3);
                else dot_chunk(wv[j], xs + c * 32, a0, a1);
            }
        }
    }
    const int part = (a0 + a1) + (a2 + a3);

    // 4. epilogue: lane r < RPW finishes row row0 + r
    int acc = 0;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int t = row_isum<LPR>(part, r) >> 4;
        if (lane == r) acc = t;
    }
    const int r = row0 + lane;
    if (lane < RPW && r < p.rows) {
        const float v = (float(acc) * act) * es;
        if (p.acc_out) p.acc_out[r] = acc;
        if constexpr (EPI == EPI_STORE) {
            p.out[r] = v;
        } else {
            if (p.out_aux) p.out_aux[r] = v;
            p.out[r] = ex + v;
        }
    }
}

// Plain fallback for the reference-signature entry when the fast path's
// layout conditions (width % 32 == 0, 16-byte aligned rows) do not hold:
// one wave per row, byte loads, same integer result and epilogue.
__global__ __launch_bounds__(kBlock) void gemv_generic_kernel(
    const int8_t* x, const uint8_t* w, const float* ws, float act, float* out, int rows,
    int width, int32_t* acc_out)
{
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * (kBlock / kWave) + wave;
    if (row >= rows) return;
    const int half = width >> 1;
    const uint8_t* wr = w + size_t(row) * size_t(half);
    int acc = 0;
    for (int j = lane; j < half; j += kWave) {
        const uint8_t b = wr[j];
        const int lo = int(int8_t(uint8_t(b << 4))) >> 4;
        const int hi = int(int8_t(b)) >> 4;
        acc += lo * int(x[2 * j]) + hi * int(x[2 * j + 1]);
    }
    acc = wave_isum64(acc);
    if (lane == 0) {
        out[row] = (float(acc) * act) * ws[row];
        if (acc_out) acc_out[row] = acc;
    }
}

// Single-block spec quantizer (hq_quantize_activation).
__global__ __launch_bounds__(kBlock) void quantize_kernel(const float* x, int n, int8_t* q,
                                                          float* act_out)
{
    __shared__ float red[4];
    float amax = 0.0f;
    for (int i = threadIdx.x; i < n; i += kBlock) amax = fmaxf(amax, fabsf(x[i]));
    amax = block_max_nonneg(amax, red);
    amax = fmaxf(amax, 1e-5f);
    const float inv = 127.0f / amax;
    for (int i = threadIdx.x; i < n; i += kBlock) q[i] = quant_i8(x[i], inv);
    if (threadIdx.x == 0) *act_out = amax / 127.0f;
}

// Single-block spec RMSNorm (hq_rmsnorm): 256-lane fmaf partials, tree.
__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(const float* x, const float* gamma,
                                                         float* y, int n, float eps)
{
    __shared__ float red[kBlock];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += kBlock) ss = __builtin_fmaf(x[i], x[i], ss);
    const float total = block_tree_sum256(ss, red);
    const float r = __builtin_sqrtf(total / float(n) + eps);
    for (int i = threadIdx.x; i < n; i += kBlock) y[i] = (x[i] / r) * gamma[i];
}

// Device argmax with np.argmax's order (hq_argmax): each block reduces 4096
// values to a (value, index) partial; the last block to arrive reduces the
// partials, writes the index and re-zeroes its arrival counter.
constexpr int kArgmaxPerBlock = kBlock * 16;

__global__ __launch_bounds__(kBlock) void argmax_kernel(const float* x, int n, float* pval,
                                                        int32_t* pidx, int32_t* counter,
                                                        int32_t* out)
{
    __shared__ float sv[kBlock / kWave];
    __shared__ int si[kBlock / kWave];
    __shared__ int last_flag;
    const int tid = threadIdx.x;
    float v = -__builtin_inff();
    int idx = 0x7FFFFFFF;
    const int base = blockIdx.x * kArgmaxPerBlock;
    for (int i = base + tid; i < min(n, base + kArgmaxPerBlock); i += kBlock)
        if (argmax_better(x[i], i, v, idx)) { v = x[i]; idx = i; }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const int oi = __shfl_xor(idx, o, kWave);
        if (argmax_better(ov, oi, v, idx)) { v = ov; idx = oi; }
    }
    if ((tid & (kWave - 1)) == 0) { sv[tid / kWave] = v; si[tid / kWave] = idx; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kBlock / kWave; ++w)
            if (argmax_better(sv[w], si[w], v, idx)) { v = sv[w]; idx = si[w]; }
        publish_f(pval + blockIdx.x, v);
        publish_i(pidx + blockIdx.x, idx);
        wait_all_memory();
        last_flag = last_block_ticket(counter, blockIdx.x, gridDim.x);
    }
    __syncthreads();
    if (!last_flag) return;
    v = -__builtin_inff();
    idx = 0x7FFFFFFF;
    for (int b = tid; b < int(gridDim.x); b += kBlock) {
        const float bv = read_f(pval + b);
        const int bi = read_i(pidx + b);
        if (argmax_better(bv, bi, v, idx)) { v = bv; idx = bi; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const int oi = __shfl_xor(idx, o, kWave);
        if (argmax_better(ov, oi, v, idx)) { v = ov; idx = oi; }
    }
    __syncthreads();
    if ((tid & (kWave - 1)) == 0) { sv[tid / kWave] = v; si[tid / kWave] = idx; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kBlock / kWave; ++w)
            if (argmax_better(sv[w], si[w], v, idx)) { v = sv[w]; idx = si[w]; }
        *out = idx;
    }
}

// ---------------------------------------------------------------------------
// host-side dispatch
// ---------------------------------------------------------------------------
template <int LPR, int MAXC, int XJ, int PRO, int EPI, bool PERSIST = false>
static hipError_t launch(const GemvParams& p, int blocks, hipStream_t s)
{
    hipLaunchKernelGGL((gemv_kernel<LPR, MAXC, XJ, PRO, EPI, PERSIST>), dim3(blocks), dim3(kBlock),
                       size_t(p.width), s, p);
    return hipGetLastError();
}

// XJ (register-resident activations per thread) is picked from the width.
template <int LPR, int MAXC, int PRO, int EPI, bool PERSIST = false>
static hipError_t launch_xj(const GemvParams& p, int blocks, hipStream_t s)
{
    if (PRO == PRO_I8) return launch<LPR, MAXC, 1, PRO, EPI, PERSIST>(p, blocks, s);
    if (p.width <= 10 * kBlock) return launch<LPR, MAXC, 10, PRO, EPI, PERSIST>(p, blocks, s);
    if (p.width <= 16 * kBlock) return launch<LPR, MAXC, 16, PRO, EPI, PERSIST>(p, blocks, s);
    return launch<LPR, MAXC, 40, PRO, EPI, PERSIST>(p, blocks, s);
}

constexpr int kMaxWidth = 40 * kBlock;   // 10240: register-resident activation limit

// Compute units of the current device (cached per device; 0 on error).
static int device_cus()
{
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = -1;
        cus[dev] = n;
    }
    return cus[dev] > 0 ? cus[dev] : 0;
}

// gemv_rr_kernel grid: tiles of 64/LPR rows, tpb = ceil(tiles / CUs) per
// block, one per wave, at least 4 (the prologue's waves) and at most 16, so
// one block per CU from 4 * CUs up to 16 * CUs tiles.  Returns the blocks
// (0 when the device cannot be queried).
static int rr_blocks(int rows, int lpr, int& tpb)
{
    const int cus = device_cus();
    if (cus == 0) return 0;
    const int rpw = kWave / lpr;
    const int tiles = (rows + rpw - 1) / rpw;
    tpb = min(16, max(4, (tiles + cus - 1) / cus));
    return (tiles + tpb - 1) / tpb;
}

template <int LPR, int C, int XJ, int PRO, int EPI>
static hipError_t launch_rr(const GemvParams& p, hipStream_t s)
{
    int tpb = 0;
    const int blocks = rr_blocks(p.rows, LPR, tpb);
    if (blocks == 0) return hipErrorInvalidDevice;
    hipLaunchKernelGGL((gemv_rr_kernel<LPR, C, XJ, PRO, EPI>), dim3(blocks), dim3(tpb * kWave),
                       size_t(p.width), s, p, tpb);
    return hipGetLastError();
}

template <int LPR, int C, int PRO, int EPI>
static hipError_t launch_rr_xj(const GemvParams& p, hipStream_t s)
{
    if (PRO == PRO_I8) return launch_rr<LPR, C, 1, PRO, EPI>(p, s);
    if (p.width <= 10 * kBlock) return launch_rr<LPR, C, 10, PRO, EPI>(p, s);
    if (p.width <= 16 * kBlock) return launch_rr<LPR, C, 16, PRO, EPI>(p, s);
    return launch_rr<LPR, C, 40, PRO, EPI>(p, s);
}

// Lanes per row of the reference-ABI GEMVs by row width: every lane holds
// up to 10 chunks of its row (rows past 64 * 10 chunks take further
// batches).
template <int PRO>
static hipError_t launch_rr_width(const GemvParams& p, hipStream_t s)
{
    const int chunks = p.width >> 5;
    if (chunks <= 10 * 8) return launch_rr_xj<8, 10, PRO, EPI_STORE>(p, s);
    if (chunks <= 10 * 16) return launch_rr_xj<16, 10, PRO, EPI_STORE>(p, s);
    if (chunks <= 10 * 32) return launch_rr_xj<32, 10, PRO, EPI_STORE>(p, s);
    return launch_rr_xj<64, 10, PRO, EPI_STORE>(p, s);
}

// Step GEMV layouts (the five-kernels-per-layer form):
//   qkv      K 2560  gemv_rr_kernel, 16 lanes/row, 5 chunks/lane   256 blocks
//   o        K 4096  gemv_rr_kernel, 32 lanes/row, 4 chunks/lane   256 blocks
//   down     K 9728  gemv_rr_kernel, 64 lanes/row, 5 chunks/lane   256 blocks
//            (qkv 5.19 -> 4.39 us, o 4.63 -> 4.21, down 8.00 -> 7.52 against
//            gemv_kernel's 256-thread tiles)
//   gate_up  K 2560  gemv_kernel, 8 lanes/row, 10 chunks/lane, 608 tiles (16 gate/up pairs)
//   LM head  K 2560  gemv_kernel, 8 lanes/row, 10 chunks/lane, 4748 tiles, persistent:
//            2 blocks per CU loop over the tiles
constexpr int kGateLPR = 8, kHeadLPR = 8;
constexpr int kPersistBlocks = 512;   // LM head: 39.0 us; 256 / 768 / 1024 blocks measured 47.4 / 40.2 / 45.4

static int rows_per_tile(int lpr) { return 4 * (kWave / lpr); }
static bool lm_head_persistent(int width) { return width <= 10 * kHeadLPR * 32; }

int step_gemv_blocks(StepGemv kind, int rows, int half_rows, int width)
{
    auto tiles = [](int n, int per) { return (n + per - 1) / per; };
    int tpb = 0;
    switch (kind) {
    case StepGemv::Qkv: return rr_blocks(rows, 16, tpb);
    case StepGemv::OResidual: return rr_blocks(rows, 32, tpb);
    case StepGemv::GateUpSwiglu: return tiles(half_rows, rows_per_tile(kGateLPR) / 2);
    case StepGemv::DownResidual: return rr_blocks(rows, 64, tpb);
    case StepGemv::LmHead: {
        const int t = tiles(rows, rows_per_tile(kHeadLPR));
        if (!lm_head_persistent(width)) return t;
        return t < kPersistBlocks ? t : kPersistBlocks;
    }
    }
    return 0;
}

hipError_t launch_step_gemv(StepGemv kind, const GemvParams& p, hipStream_t s)
{
    const int blocks = step_gemv_blocks(kind, p.rows, p.half_rows, p.width);
    switch (kind) {
    case StepGemv::Qkv: return launch_rr_xj<16, 5, PRO_RMSNORM, EPI_STORE>(p, s);
    case StepGemv::OResidual: return launch_rr_xj<32, 4, PRO_QUANT, EPI_RESIDUAL>(p, s);
    case StepGemv::GateUpSwiglu: return launch_xj<kGateLPR, 10, PRO_RMSNORM, EPI_SWIGLU>(p, blocks, s);
    case StepGemv::DownResidual: return launch_rr_xj<64, 5, PRO_QUANT, EPI_RESIDUAL>(p, s);
    case StepGemv::LmHead:
        if (lm_head_persistent(p.width))   // one weight batch per tile
            return launch_xj<kHeadLPR, 10, PRO_RMSNORM, EPI_ARGMAX, true>(p, blocks, s);
        return launch_xj<kHeadLPR, 10, PRO_RMSNORM, EPI_ARGMAX, false>(p, blocks, s);
    }
    return hipErrorInvalidValue;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace hq

using namespace hq;

extern "C" int hq_int4_i8_gemv(const int8_t* x, const uint8_t* weights, const float* scales,
                               float activation_scale, float* output, int rows, int width,
                               void* stream)
{
    if (rows < 0 || width <= 0 || (width & 1)) return HQ_ERR_ARG;
    if (rows == 0) return HQ_OK;
    if (!x || !weights || !scales || !output) return HQ_ERR_ARG;
    if (width > 32768) return HQ_ERR_ARG;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    if ((width & 31) == 0 && aligned16(weights)) {
        GemvParams p{};
        p.w = weights; p.ws = scales; p.rows = rows; p.width = width;
        p.xq = x; p.act_scale = activation_scale; p.out = output;
        e = launch_rr_width<PRO_I8>(p, s);
    } else {
        const int per = kBlock / kWave;
        hipLaunchKernelGGL(gemv_generic_kernel, dim3((rows + per - 1) / per), dim3(kBlock), 0, s,
                           x, weights, scales, activation_scale, output, rows, width,
                           static_cast<int32_t*>(nullptr));
        e = hipGetLastError();
    }
    return e == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}

extern "C" int hq_quant_int4_gemv(const float* x, const uint8_t* weights, const float* scales,
                                  float* output, int rows, int width, int8_t* q_out,
                                  float* act_scale_out, int32_t* acc_out, void* stream)
{
    if (rows < 0 || width <= 0 || (width & 1)) return HQ_ERR_ARG;
    if (rows == 0) return HQ_OK;
    if (!x || !weights || !scales || !output) return HQ_ERR_ARG;
    if (width > kMaxWidth) return HQ_ERR_ARG;
    if ((width & 31) != 0 || !aligned16(weights)) return HQ_ERR_ALIGN;
    GemvParams p{};
    p.w = weights; p.ws = scales; p.rows = rows; p.width = width;
    p.xf = x; p.out = output; p.q_out = q_out; p.act_out = act_scale_out; p.acc_out = acc_out;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // one block per CU, each with the same number of rows (the prologue is
    // done once per CU)
    const hipError_t e = launch_rr_width<PRO_QUANT>(p, s);
    return e == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}

extern "C" int hq_quantize_activation(const float* x, int n, int8_t* q, float* act_scale,
                                      void* stream)
{
    if (n <= 0 || !x || !q || !act_scale) return HQ_ERR_ARG;
    hipLaunchKernelGGL(quantize_kernel, dim3(1), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), x, n, q, act_scale);
    return hipGetLastError() == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}

extern "C" int hq_rmsnorm(const float* x, const float* gamma, float* y, int n, float eps,
                          void* stream)
{
    if (n <= 0 || !x || !gamma || !y) return HQ_ERR_ARG;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), x, gamma, y, n, eps);
    return hipGetLastError() == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}

extern "C" size_t hq_argmax_workspace_bytes(int n)
{
    if (n <= 0) return 0;
    const size_t blocks = (size_t(n) + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
    // arrival counters first, then the partials
    return ((size_t(ticket_words(int(blocks))) * 4 + 255) & ~size_t(255)) + blocks * 8;
}

extern "C" int hq_argmax(const float* x, int n, int32_t* out_index, void* workspace, void* stream)
{
    if (n <= 0 || !x || !out_index || !workspace) return HQ_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return HQ_ERR_ALIGN;
    const int blocks = (n + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
    char* ws = static_cast<char*>(workspace);
    const size_t off = (size_t(ticket_words(blocks)) * 4 + 255) & ~size_t(255);
    int32_t* counter = reinterpret_cast<int32_t*>(ws);
    float* pval = reinterpret_cast<float*>(ws + off);
    int32_t* pidx = reinterpret_cast<int32_t*>(ws + off + size_t(blocks) * 4);
    hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), x, n, pval, pidx, counter, out_index);
    return hipGetLastError() == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}
