// attn_pack.hip -- fp32/bf16 (BH,S,D) rows -> the bf16 operand layouts the
// MFMA kernels read.
//
// Two layouts per source tensor X (BH,S,D), S padded to Sp (a multiple of 64,
// pad rows zero):
//   row  Xb (BH,Sp,D) bf16, row-major: an MFMA operand whose lanes each take
//        one row of X and 8 consecutive elements along D.
//   tr   Xt (BH,D,Sp) bf16, transposed, with the positions inside every group
//        of 16 permuted by vt_pos: an MFMA operand that contracts over the
//        sequence axis against P, dS (or their transposes) taken straight from
//        an accumulator, so each lane's 8 k-values are one 16-byte read.
// One launch packs up to two sources, each times a factor (1, or the sign of
// the scale for the backward's Q); either output of a source may be null.
//
// HBM-bound: per element 4 (f32) or 2 (bf16) bytes read and 2 bytes written
// per output layout. A workgroup owns 64 rows of one (b,h) slice:
//   phase 1: each lane reads 4 consecutive elements (16 B of f32, lanes along
//            D, fully coalesced), converts to bf16, writes them to Xb (8 B
//            per lane, coalesced) and, for Xt, to a row-major LDS tile;
//   phase 2: (Xt only) a lane owns 4 consecutive d and 8 output positions:
//            eight 8-byte LDS reads (4 d of one row each), a register
//            transpose, and four 16-byte stores; 8 consecutive lanes write one
//            whole 128-byte segment of an Xt row.
#include "common.h"
#include "kernels.h"

namespace gonn {

// grid (Sp/64, BH, nsrc), 256 threads.
template <typename T, int D>
__global__ __launch_bounds__(256) void pack_kernel(PackParams p) {
    constexpr int BN = 64;
    constexpr int TS = D + 4;  // LDS row stride (bf16): 8-byte rows, spread banks
    __shared__ __attribute__((aligned(16))) bf16 tile[BN * TS];
    const int tid = threadIdx.x;
    const int kt = blockIdx.x, bh = blockIdx.y, which = blockIdx.z;
    const T* src = (const T*)p.src[which];
    bf16* row = (bf16*)p.row[which];
    bf16* tr = (bf16*)p.tr[which];
    const int S = p.S, Sp = p.Sp;
    const float mul = p.mul[which];
    const size_t src0 = (size_t)bh * S * D;

    constexpr int CH = BN * D / 4;  // 4-element chunks
    constexpr int NC = CH / 256;     // per thread
    // All of this thread's loads are issued before any store, so NC loads
    // are in flight per lane.
    float v[NC][4];
    for (int n = 0; n < NC; n++) {
        const int c = tid + n * 256;
        const int r = c / (D / 4), col = (c % (D / 4)) * 4;
        const int key = kt * BN + r;
        const int keyc = key < S ? key : S - 1;  // rows past S become zero below
        const T* sp = src + src0 + (size_t)keyc * D + col;
        if constexpr (sizeof(T) == 4) {
            const f32x4 a = __builtin_nontemporal_load((const f32x4*)sp);
            for (int i = 0; i < 4; i++) v[n][i] = a[i];
        } else {
            const uint2 a = *(const uint2*)sp;
            v[n][0] = __uint_as_float(a.x << 16);
            v[n][1] = __uint_as_float(a.x & 0xffff0000u);
            v[n][2] = __uint_as_float(a.y << 16);
            v[n][3] = __uint_as_float(a.y & 0xffff0000u);
        }
    }
    typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
    for (int n = 0; n < NC; n++) {
        const int c = tid + n * 256;
        const int r = c / (D / 4), col = (c % (D / 4)) * 4;
        const int key = kt * BN + r;
        bf16x4 b;
        for (int i = 0; i < 4; i++) b[i] = to_bf16(key < S ? v[n][i] * mul : 0.f);
        if (row) *(bf16x4*)(row + ((size_t)bh * Sp + key) * D + col) = b;
        if (tr) *(bf16x4*)(tile + r * TS + col) = b;
    }
    if (!tr) return;  // uniform for the workgroup
    __syncthreads();
    // Lane -> (j: 8 output positions, d4: 4 consecutive d).
    constexpr int NT = (D / 4) * 8;  // tasks
    if (tid >= NT) return;
    const int j = tid & 7, d4 = tid >> 3;
    const int grp = (j >> 1) * 16;
    uint2 w[8];  // w[i] = bf16 of d = 4*d4 .. 4*d4+3 for the key at position i
    for (int i = 0; i < 8; i++) {
        const int key = grp + vt_pos((j & 1) * 8 + i);
        w[i] = *(const uint2*)(tile + key * TS + 4 * d4);
    }
    for (int r = 0; r < 4; r++) {
        // output row d = 4*d4 + r: 8 bf16, component r of each w[i]
        u32x4 o;
        for (int q = 0; q < 4; q++) {
            const uint32_t a = (r < 2) ? w[2 * q].x : w[2 * q].y;
            const uint32_t b = (r < 2) ? w[2 * q + 1].x : w[2 * q + 1].y;
            o[q] = (r & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
        }
        *(u32x4*)(tr + ((size_t)bh * D + 4 * d4 + r) * Sp + kt * BN + j * 8) = o;
    }
}

hipError_t launch_pack(const PackParams& p, int nsrc, int in_bf16, int BH, int D, hipStream_t s) {
    if (nsrc < 1 || nsrc > 2 || p.Sp % 64 != 0) return hipErrorInvalidValue;
    dim3 grid(p.Sp / 64, BH, nsrc);
    if (D == 64) {
        if (in_bf16) pack_kernel<bf16, 64><<<grid, 256, 0, s>>>(p);
        else pack_kernel<float, 64><<<grid, 256, 0, s>>>(p);
    } else if (D == 128) {
        if (in_bf16) pack_kernel<bf16, 128><<<grid, 256, 0, s>>>(p);
        else pack_kernel<float, 128><<<grid, 256, 0, s>>>(p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gonn
