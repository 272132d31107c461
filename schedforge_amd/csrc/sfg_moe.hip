// sfg_moe.hip -- MoE routing pipeline for gfx950:
//   Router -> Softmax -> TopK   (route_topk, moe_compiler.cpp:412-455)
//   Histogram -> PrefixSum -> Segmented Dispatch (dispatch_tokens, 496-528)
//   weighted combine (219-226) fused with the FFN residual (decoder_compiler.cpp:277).
// The grouped expert GEMMs run on the GEMM family (sfg_gemm.hip) with the
// dispatch offsets as device-side group bounds and token_ids as the A gather.
//
// Integer outputs (ids, counts, offsets, token_ids, route_slots, positions)
// are exact: logits are sequential fp32 FMA chains in feature order (the order
// the reference's scalar loop accumulates), selection compares logits with ties
// to the lower expert index, and the dispatch rank of an assignment is the
// number of earlier (token, slot) assignments routed to the same expert.
#include "sfg_kernels.hpp"

namespace sfg {

// One thread per (token, expert) chain; the block then runs softmax + top-k for
// its tokens with one thread per token.  E <= 256, top_k <= 8.  The chain runs
// over features in order (bit-identical to a sequential fp32 FMA loop).
// Operands are staged through LDS in 512-feature chunks (x as [token][f], the
// router transposed to [e][f]) and fed to the chain from registers 16 features
// at a time, the next 16 already in flight; the next chunk's global loads are
// held in registers while the current chunk's chain runs.
// Softmax over all experts (max-shifted), top-k by logit (slot 0 the largest;
// ties to the lower expert index: a strictly larger logit replaces the pick),
// selected probabilities renormalised to sum 1 (moe_compiler.cpp:429-452).
__device__ void route_select(const float* lg, int experts, int top_k, int tok, int32_t* __restrict__ ids,
                             float* __restrict__ weights) {
    float maximum = -INFINITY;
    for (int j = 0; j < experts; ++j) maximum = fmaxf(maximum, lg[j]);
    float denom = 0.f;
    for (int j = 0; j < experts; ++j) denom += expf(lg[j] - maximum);
    uint32_t taken[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // bitmask over <= 256 experts
    int sel[8];
    float selected = 0.f;
    for (int s = 0; s < top_k; ++s) {
        int best = -1;
        for (int j = 0; j < experts; ++j) {
            if (taken[j >> 5] & (1u << (j & 31))) continue;
            if (best < 0 || lg[j] > lg[best]) best = j;
        }
        taken[best >> 5] |= 1u << (best & 31);
        sel[s] = best;
        selected += expf(lg[best] - maximum) / denom;
    }
    for (int s = 0; s < top_k; ++s) {
        const int j = sel[s];
        ids[static_cast<int64_t>(tok) * top_k + s] = j;
        weights[static_cast<int64_t>(tok) * top_k + s] = (expf(lg[j] - maximum) / denom) / selected;
    }
}

constexpr int kRouteChunk = 512;
constexpr int kRouteTokens = 8;        // tokens per workgroup: 64 chains, one full wave (measured 4% faster than 4 on C3 and C5)
constexpr int kRouteMaxExperts = 8;    // staged path; larger E uses the direct chain
constexpr int kRouteBlock = 16;        // chain operands per register block
// Floats of padding per staged row: room for one block read past the chunk,
// and a row stride of 532 floats puts the eight expert rows of one b128 read
// on disjoint banks.
constexpr int kRoutePad = 20;
static_assert(kRoutePad >= kRouteBlock && kRouteChunk % (2 * kRouteBlock) == 0, "router staging");
constexpr int kRouteLoads = (kRouteTokens * kRouteChunk + kRouteChunk * kRouteMaxExperts) / 256 / 4;

__global__ __launch_bounds__(256) void moe_router_kernel(
    const float* __restrict__ x, const float* __restrict__ router, const float* __restrict__ bias,
    int tokens, int hidden, int experts, int top_k, int32_t* __restrict__ ids,
    float* __restrict__ weights) {
    __shared__ float logits[256];
    __shared__ __attribute__((aligned(16))) float sx[2][kRouteTokens][kRouteChunk + kRoutePad];
    __shared__ __attribute__((aligned(16))) float sw[2][kRouteMaxExperts][kRouteChunk + kRoutePad];
    const bool staged = experts <= kRouteMaxExperts && (hidden % kRouteChunk) == 0;
    const int per_block = staged ? kRouteTokens : min(kRouteTokens, 256 / experts);
    const int t_local = threadIdx.x / experts;
    const int e = threadIdx.x % experts;
    const int t0 = blockIdx.x * per_block;
    const int t = t0 + t_local;
    const bool active = t_local < per_block && t < tokens;
    float acc = 0.f;
    if (staged) {
        // Each thread moves kRouteLoads float4 per chunk: x rows first, then the
        // router slice [f][e] (contiguous in memory) scattered to sw[e][f].
        const int x_vecs = kRouteTokens * kRouteChunk / 4;
        const int w_vecs = kRouteChunk * experts / 4;
        float4 reg[kRouteLoads];
        // LDS destinations of the router values this thread moves: the same
        // for every chunk, so the divisions by `experts` run once.
        int woff[kRouteLoads][4];
#pragma unroll
        for (int i = 0; i < kRouteLoads; ++i) {
            const int flat = 4 * (static_cast<int>(threadIdx.x) + 256 * i - x_vecs);  // = f * experts + e
#pragma unroll
            for (int j = 0; j < 4; ++j)
                woff[i][j] = flat + j >= 0 ? ((flat + j) % experts) * (kRouteChunk + kRoutePad) + (flat + j) / experts : 0;
        }
        auto fetch = [&](int f0) {
#pragma unroll
            for (int i = 0; i < kRouteLoads; ++i) {
                const int v = threadIdx.x + 256 * i;
                float4 val = make_float4(0.f, 0.f, 0.f, 0.f);
                if (v < x_vecs) {
                    const int tt = v / (kRouteChunk / 4), f4 = v % (kRouteChunk / 4);
                    if (t0 + tt < tokens)
                        val = *reinterpret_cast<const float4*>(x + static_cast<int64_t>(t0 + tt) * hidden + f0 + 4 * f4);
                } else if (v - x_vecs < w_vecs) {
                    val = *reinterpret_cast<const float4*>(router + static_cast<int64_t>(f0) * experts + 4 * (v - x_vecs));
                }
                reg[i] = val;
            }
        };
        auto stash = [&](int buf) {
#pragma unroll
            for (int i = 0; i < kRouteLoads; ++i) {
                const int v = threadIdx.x + 256 * i;
                if (v < x_vecs) {
                    const int tt = v / (kRouteChunk / 4), f4 = v % (kRouteChunk / 4);
                    *reinterpret_cast<float4*>(&sx[buf][tt][4 * f4]) = reg[i];
                } else if (v - x_vecs < w_vecs) {
                    float* swb = &sw[buf][0][0];
                    swb[woff[i][0]] = reg[i].x;
                    swb[woff[i][1]] = reg[i].y;
                    swb[woff[i][2]] = reg[i].z;
                    swb[woff[i][3]] = reg[i].w;
                }
            }
        };
        fetch(0);
        stash(0);
        __syncthreads();
        int buf = 0;
        for (int f0 = 0; f0 < hidden; f0 += kRouteChunk) {
            const bool more = f0 + kRouteChunk < hidden;
            if (more) fetch(f0 + kRouteChunk);
            if (active) {
                const float* xr = sx[buf][t_local];
                const float* wr = sw[buf][e];
                float xa[kRouteBlock], wa[kRouteBlock], xb[kRouteBlock], wb[kRouteBlock];
#pragma unroll
                for (int j = 0; j < kRouteBlock; j += 4) {
                    *reinterpret_cast<float4*>(&xa[j]) = *reinterpret_cast<const float4*>(xr + j);
                    *reinterpret_cast<float4*>(&wa[j]) = *reinterpret_cast<const float4*>(wr + j);
                }
#pragma unroll
                for (int f = 0; f < kRouteChunk; f += 2 * kRouteBlock) {
#pragma unroll
                    for (int j = 0; j < kRouteBlock; j += 4) {
                        *reinterpret_cast<float4*>(&xb[j]) = *reinterpret_cast<const float4*>(xr + f + kRouteBlock + j);
                        *reinterpret_cast<float4*>(&wb[j]) = *reinterpret_cast<const float4*>(wr + f + kRouteBlock + j);
                    }
#pragma unroll
                    for (int j = 0; j < kRouteBlock; ++j) acc = __builtin_fmaf(xa[j], wa[j], acc);
                    // unconditional: the last block's read lands in the row
                    // padding and is unused, and the two register sets
                    // alternate without copies
#pragma unroll
                    for (int j = 0; j < kRouteBlock; j += 4) {
                        *reinterpret_cast<float4*>(&xa[j]) = *reinterpret_cast<const float4*>(xr + f + 2 * kRouteBlock + j);
                        *reinterpret_cast<float4*>(&wa[j]) = *reinterpret_cast<const float4*>(wr + f + 2 * kRouteBlock + j);
                    }
#pragma unroll
                    for (int j = 0; j < kRouteBlock; ++j) acc = __builtin_fmaf(xb[j], wb[j], acc);
                }
            }
            __syncthreads();
            if (more) stash(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }
    } else if (active) {
        const float* xr = x + static_cast<int64_t>(t) * hidden;
        for (int f = 0; f < hidden; ++f)
            acc = __builtin_fmaf(xr[f], router[static_cast<int64_t>(f) * experts + e], acc);
    }
    if (active) {
        if (bias) acc = acc + bias[e];
        logits[t_local * experts + e] = acc;
    }
    __syncthreads();
    if (static_cast<int>(threadIdx.x) >= per_block) return;
    const int tok = blockIdx.x * per_block + threadIdx.x;
    if (tok >= tokens) return;
    route_select(logits + threadIdx.x * experts, experts, top_k, tok, ids, weights);
}

int launch_moe_router(const float* x, const float* router, const float* bias, int64_t tokens,
                      int64_t hidden, int64_t experts, int64_t top_k, int32_t* ids,
                      float* weights, hipStream_t stream) {
    if (experts <= 0 || experts > 256 || top_k <= 0 || top_k > 8 || top_k > experts)
        return SFG_ERR_UNSUPPORTED;
    const int per_block = experts <= kRouteMaxExperts
        ? kRouteTokens : static_cast<int>(256 / experts < kRouteTokens ? 256 / experts : kRouteTokens);
    const dim3 grid(static_cast<unsigned>((tokens + per_block - 1) / per_block));
    moe_router_kernel<<<grid, 256, 0, stream>>>(x, router, bias, static_cast<int>(tokens),
                                                static_cast<int>(hidden), static_cast<int>(experts),
                                                static_cast<int>(top_k), ids, weights);
    return SFG_OK;
}

// Single workgroup of 1024 threads: histogram (LDS atomics), exclusive prefix
// over experts, then a stable scatter: assignments are visited in chunks of
// 1024 in (token, slot) order; inside a wave the rank among equal experts is a
// popcount of the matching-lanes ballot below the lane, across waves an
// exclusive scan of per-wave counts, across chunks a running cursor.
__global__ __launch_bounds__(1024) void moe_dispatch_kernel(
    const int32_t* __restrict__ ids, const float* __restrict__ weights, int total, int experts,
    int top_k, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ token_ids, int32_t* __restrict__ route_slots,
    float* __restrict__ routing_weights, int32_t* __restrict__ position) {
    __shared__ int s_count[256];
    __shared__ int s_cursor[256];
    __shared__ int s_wave[16][256];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < experts; e += 1024) s_count[e] = 0;
    __syncthreads();
    for (int a = tid; a < total; a += 1024) {
        const int e = ids[a];
        if (e >= 0 && e < experts) atomicAdd(&s_count[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int e = 0; e < experts; ++e) {
            offsets[e] = run;
            s_cursor[e] = run;
            counts[e] = s_count[e];
            run += s_count[e];
        }
        offsets[experts] = run;
    }
    __syncthreads();
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = 0; base < total; base += 1024) {
        const int a = base + tid;
        const bool active = a < total;
        const int e = active ? ids[a] : -1;
        for (int j = tid; j < 16 * experts; j += 1024) s_wave[j / experts][j % experts] = 0;
        __syncthreads();
        // Per-wave ranks: peel off one expert value per iteration.
        int rank = 0;
        uint64_t pending = __ballot(active && e >= 0 && e < experts);
        while (pending) {
            const int leader = __ffsll(static_cast<unsigned long long>(pending)) - 1;
            const int le = __shfl(e, leader, 64);
            const uint64_t match = __ballot(active && e == le);
            if (active && e == le) rank = __popcll(match & below);
            if (lane == 0) s_wave[wave][le] = __popcll(match);
            pending &= ~match;
        }
        __syncthreads();
        // Exclusive scan across the 16 waves, per expert; advance cursors.
        for (int x = tid; x < experts; x += 1024) {
            int run = s_cursor[x];
            for (int w = 0; w < 16; ++w) {
                const int c = s_wave[w][x];
                s_wave[w][x] = run;
                run += c;
            }
            s_cursor[x] = run;
        }
        __syncthreads();
        if (active && e >= 0 && e < experts) {
            const int dst = s_wave[wave][e] + rank;
            token_ids[dst] = a / top_k;
            route_slots[dst] = a % top_k;
            routing_weights[dst] = weights[a];
            position[a] = dst;
        } else if (active) {
            position[a] = -1;  // expert id out of range: the combine skips it
        }
        __syncthreads();
    }
}

// Same dispatch for at most kDispExperts experts and kDispChunks x 1024
// assignments (the decode and prefill MoE shapes): every assignment's expert
// and weight is loaded once, up front, into registers; each wave ranks its 64
// assignments of every chunk by ballot; then (chunk, expert) threads turn the
// per-wave counts into offsets, expert threads the per-chunk counts, and one
// thread the per-expert totals -- five barriers for the whole dispatch instead
// of four per chunk.  Destinations are the same as moe_dispatch_kernel's
// (stable in (token, slot) order inside each expert).
constexpr int kDispChunks = 8;
constexpr int kDispExperts = 16;

__global__ __launch_bounds__(1024) void moe_dispatch_reg_kernel(
    const int32_t* __restrict__ ids, const float* __restrict__ weights, int total, int experts,
    int top_k, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ token_ids, int32_t* __restrict__ route_slots,
    float* __restrict__ routing_weights, int32_t* __restrict__ position) {
    __shared__ int s_wave[kDispChunks][16][kDispExperts];   // count, then offset inside the chunk
    __shared__ int s_chunk_cnt[kDispChunks][kDispExperts];
    __shared__ int s_chunk_off[kDispChunks][kDispExperts];  // offset inside the expert
    __shared__ int s_count[kDispExperts];
    __shared__ int s_base[kDispExperts];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int chunks = (total + 1023) / 1024;
    int e_c[kDispChunks];
    float w_c[kDispChunks];
#pragma unroll
    for (int c = 0; c < kDispChunks; ++c) {
        const int a = c * 1024 + tid;
        const bool act = a < total;
        e_c[c] = act ? ids[a] : -1;
        w_c[c] = act ? weights[a] : 0.f;
    }
    // Per-wave ranks of every chunk: peel off one expert value per iteration.
    // A wave zeroes and then fills only its own counters, in program order.
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int rank_c[kDispChunks];
#pragma unroll
    for (int c = 0; c < kDispChunks; ++c) {
        rank_c[c] = 0;
        if (c >= chunks) continue;
        const int e = e_c[c];
        const bool valid = e >= 0 && e < experts;
        if (lane < kDispExperts) s_wave[c][wave][lane] = 0;
        uint64_t pending = __ballot(valid);
        while (pending) {
            const int leader = __ffsll(static_cast<unsigned long long>(pending)) - 1;
            const int le = __builtin_amdgcn_readlane(e, leader);  // leader is wave-uniform
            const uint64_t match = __ballot(valid && e == le);
            if (valid && e == le) rank_c[c] = __popcll(match & below);
            if (lane == 0) s_wave[c][wave][le] = __popcll(match);
            pending &= ~match;
        }
    }
    __syncthreads();
    // (chunk, expert): exclusive prefix over the 16 waves, chunk total
    if (tid < chunks * kDispExperts) {
        const int c = tid / kDispExperts, x = tid % kDispExperts;
        int v[16];
#pragma unroll
        for (int w = 0; w < 16; ++w) v[w] = s_wave[c][w][x];
        int run = 0;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            s_wave[c][w][x] = run;
            run += v[w];
        }
        s_chunk_cnt[c][x] = run;
    }
    __syncthreads();
    // expert: exclusive prefix over the chunks, expert total (the histogram)
    if (tid < experts) {
        int run = 0;
        for (int c = 0; c < chunks; ++c) {
            s_chunk_off[c][tid] = run;
            run += s_chunk_cnt[c][tid];
        }
        s_count[tid] = run;
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int e = 0; e < experts; ++e) {
            offsets[e] = run;
            s_base[e] = run;
            counts[e] = s_count[e];
            run += s_count[e];
        }
        offsets[experts] = run;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kDispChunks; ++c) {
        const int e = e_c[c];
        const int a = c * 1024 + tid;
        if (c >= chunks || a >= total) continue;
        if (e < 0 || e >= experts) {
            position[a] = -1;  // expert id out of range: the combine skips it
            continue;
        }
        const int dst = s_base[e] + s_chunk_off[c][e] + s_wave[c][wave][e] + rank_c[c];
        token_ids[dst] = a / top_k;
        route_slots[dst] = a % top_k;
        routing_weights[dst] = w_c[c];
        position[a] = dst;
    }
}

int launch_moe_dispatch(const int32_t* ids, const float* weights, int64_t tokens,
                        int64_t experts, int64_t top_k, int32_t* counts, int32_t* offsets,
                        int32_t* token_ids, int32_t* route_slots, float* routing_weights,
                        int32_t* position, hipStream_t stream) {
    if (experts <= 0 || experts > 256) return SFG_ERR_UNSUPPORTED;
    const int64_t total = tokens * top_k;
    if (total > (1ll << 30)) return SFG_ERR_UNSUPPORTED;
    if (experts <= kDispExperts && total <= kDispChunks * 1024) {
        moe_dispatch_reg_kernel<<<1, 1024, 0, stream>>>(ids, weights, static_cast<int>(total),
                                                         static_cast<int>(experts), static_cast<int>(top_k),
                                                         counts, offsets, token_ids, route_slots,
                                                         routing_weights, position);
        return SFG_OK;
    }
    moe_dispatch_kernel<<<1, 1024, 0, stream>>>(ids, weights, static_cast<int>(total),
                                                 static_cast<int>(experts), static_cast<int>(top_k),
                                                 counts, offsets, token_ids, route_slots,
                                                 routing_weights, position);
    return SFG_OK;
}

size_t moe_route_workspace_bytes(int64_t tokens, int64_t experts, int64_t top_k) {
    (void)tokens; (void)experts; (void)top_k;
    return 0;
}

// out[t][f] = residual[t][f] + sum_s w[t][s] * y[position[t][s]][f], slots in
// order (the token-major order of reference_moe, moe_compiler.cpp:651-679).
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const float* __restrict__ y, const int32_t* __restrict__ position,
    const float* __restrict__ weights, const float* __restrict__ residual,
    float* __restrict__ out, int hidden, int top_k, int64_t total) {
    const int t = blockIdx.x;
    for (int f = threadIdx.x * 4; f < hidden; f += 256 * 4) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s = 0; s < top_k; ++s) {
            const float w = weights[static_cast<int64_t>(t) * top_k + s];
            const int64_t pos = position[static_cast<int64_t>(t) * top_k + s];
            if (pos < 0 || pos >= total) continue;  // corrupt index: contributes nothing
            const float4 v = *reinterpret_cast<const float4*>(y + pos * hidden + f);
            acc.x = fmaf(w, v.x, acc.x);
            acc.y = fmaf(w, v.y, acc.y);
            acc.z = fmaf(w, v.z, acc.z);
            acc.w = fmaf(w, v.w, acc.w);
        }
        const float4 r = *reinterpret_cast<const float4*>(residual + static_cast<int64_t>(t) * hidden + f);
        *reinterpret_cast<float4*>(out + static_cast<int64_t>(t) * hidden + f) =
            make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
    }
}

// top_k <= KMAX: the token's (position, weight) pairs are read once, and each
// feature block issues every assignment's row load together with the residual
// before the first wait.  Slots past top_k and invalid positions read row 0 and
// are left out of the sum, which runs over the slots in order as above.
template <int KMAX>
__global__ __launch_bounds__(256) void moe_combine_reg_kernel(
    const float* __restrict__ y, const int32_t* __restrict__ position,
    const float* __restrict__ weights, const float* __restrict__ residual,
    float* __restrict__ out, int hidden, int top_k, int64_t total) {
    const int t = blockIdx.x;
    int64_t pos[KMAX];
    float w[KMAX];
    bool ok[KMAX];
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
        const int sc = s < top_k ? s : top_k - 1;
        const int64_t ps = position[static_cast<int64_t>(t) * top_k + sc];
        w[s] = weights[static_cast<int64_t>(t) * top_k + sc];
        ok[s] = s < top_k && ps >= 0 && ps < total;  // corrupt index: contributes nothing
        pos[s] = ok[s] ? ps : 0;
    }
    for (int f = threadIdx.x * 4; f < hidden; f += 256 * 4) {
        float4 v[KMAX];
#pragma unroll
        for (int s = 0; s < KMAX; ++s) v[s] = *reinterpret_cast<const float4*>(y + pos[s] * hidden + f);
        const float4 r = *reinterpret_cast<const float4*>(residual + static_cast<int64_t>(t) * hidden + f);
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int s = 0; s < KMAX; ++s) {
            if (!ok[s]) continue;
            acc.x = fmaf(w[s], v[s].x, acc.x);
            acc.y = fmaf(w[s], v[s].y, acc.y);
            acc.z = fmaf(w[s], v[s].z, acc.z);
            acc.w = fmaf(w[s], v[s].w, acc.w);
        }
        *reinterpret_cast<float4*>(out + static_cast<int64_t>(t) * hidden + f) =
            make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
    }
}

// Hidden sizes that are not a multiple of 4: one feature per thread, the same
// slot-ordered sum.
__global__ __launch_bounds__(256) void moe_combine_scalar_kernel(
    const float* __restrict__ y, const int32_t* __restrict__ position,
    const float* __restrict__ weights, const float* __restrict__ residual,
    float* __restrict__ out, int hidden, int top_k, int64_t total) {
    const int t = blockIdx.x;
    for (int f = threadIdx.x; f < hidden; f += 256) {
        float acc = 0.f;
        for (int s = 0; s < top_k; ++s) {
            const int64_t pos = position[static_cast<int64_t>(t) * top_k + s];
            if (pos < 0 || pos >= total) continue;  // corrupt index: contributes nothing
            acc = fmaf(weights[static_cast<int64_t>(t) * top_k + s], y[pos * hidden + f], acc);
        }
        out[static_cast<int64_t>(t) * hidden + f] = residual[static_cast<int64_t>(t) * hidden + f] + acc;
    }
}

void launch_moe_combine(const float* y, const int32_t* position, const float* weights,
                        const float* residual, float* out, int64_t tokens, int64_t hidden,
                        int64_t top_k, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(tokens));
    const int h = static_cast<int>(hidden), k = static_cast<int>(top_k);
    if (hidden & 3) moe_combine_scalar_kernel<<<grid, 256, 0, stream>>>(y, position, weights, residual, out, h, k, tokens * top_k);
    else if (top_k <= 2) moe_combine_reg_kernel<2><<<grid, 256, 0, stream>>>(y, position, weights, residual, out, h, k, tokens * top_k);
    else if (top_k <= 4) moe_combine_reg_kernel<4><<<grid, 256, 0, stream>>>(y, position, weights, residual, out, h, k, tokens * top_k);
    else if (top_k <= 8) moe_combine_reg_kernel<8><<<grid, 256, 0, stream>>>(y, position, weights, residual, out, h, k, tokens * top_k);
    else moe_combine_kernel<<<grid, 256, 0, stream>>>(y, position, weights, residual, out, h, k, tokens * top_k);
}

}  // namespace sfg
