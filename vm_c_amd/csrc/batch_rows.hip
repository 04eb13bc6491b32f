// batch_rows.hip -- one (sequence, position) row per query token of a step,
// from the batch metadata vm_c's Engine uploads.
//
// The Engine (src/core/engine.cpp:653-793) lays a step's tokens out request
// by request and uploads block_tables [num_reqs][max_blocks] and seq_lens
// [num_reqs]; token_to_seq / token_positions [num_tokens] are written only
// when the step has prefill requests, and only for the prefill requests'
// tokens (:686-691, :760-766) -- a decode request's single token keeps 0 / 0.
// The ggml TurboQuant node (src/official/turboquant_kv_bridge.cpp:99-107)
// decodes num_tokens rows over those per-request arrays, which reads past
// both of them in any step with prefill tokens.  This kernel gives every
// token the row the paged prefill attention takes instead:
//   prefill token t: (token_to_seq[t], token_positions[t]);
//   decode token t:  (r, seq_lens[r] - 1) with r its request, counted from
//                    the request boundaries in token order.
// A token starts a request when it is the first token, a decode token, the
// token after a decode token, or a prefill token of another request than the
// token before it.  0 / 0 marks a decode token, except for token 0 when
// token 1 is (0, 1): then request 0 is a prefill from position 0.  (A
// one-token prefill of request 0 at position 0 reads as a decode token; both
// give position seq_lens[0] - 1 = 0.)  Rows whose request lies outside
// [0, num_reqs) get position -1 (no keys, a zero output row).
#include "vmc_common.hpp"

namespace vmc {
namespace {

constexpr int kRowThreads = 1024;

__device__ __forceinline__ bool is_decode_token(const int32_t* ts, const int32_t* tp, int t, bool first_prefill) {
    return ts[t] == 0 && tp[t] == 0 && (t > 0 || !first_prefill);
}

__global__ void __launch_bounds__(kRowThreads)
batch_rows_kernel(const int32_t* __restrict__ ts, const int32_t* __restrict__ tp,
                  const int32_t* __restrict__ seq_lens, int T, int R, int32_t* __restrict__ row_seq,
                  int32_t* __restrict__ row_pos) {
    __shared__ int wsum[kRowThreads / 64];
    __shared__ int carry;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool first_prefill = T > 1 && ts[1] == 0 && tp[1] == 1;
    if (tid == 0) carry = 0;
    __syncthreads();
    for (int base = 0; base < T; base += kRowThreads) {
        const int t = base + tid;
        const bool in = t < T;
        bool dec = false, start = false;
        if (in) {
            dec = is_decode_token(ts, tp, t, first_prefill);
            start = t == 0 || dec || is_decode_token(ts, tp, t - 1, first_prefill) || ts[t] != ts[t - 1];
        }
        const uint64_t bal = __ballot(start);
        const int incl = __popcll(bal & ((2ull << lane) - 1ull));
        if (lane == 0) wsum[wave] = __popcll(bal);
        __syncthreads();
        int req = carry + incl - 1;
        for (int w = 0; w < wave; ++w) req += wsum[w];
        if (in) {
            const int s = dec ? req : ts[t];
            const bool ok = s >= 0 && s < R;
            row_seq[t] = ok ? s : 0;
            row_pos[t] = !ok ? -1 : dec ? seq_lens[s] - 1 : tp[t];
        }
        __syncthreads();
        if (tid == 0) {
            int tot = carry;
            for (int w = 0; w < kRowThreads / 64; ++w) tot += wsum[w];
            carry = tot;
        }
        __syncthreads();
    }
}

}  // namespace
}  // namespace vmc

using namespace vmc;

extern "C" int vmc_batch_token_rows(int32_t* row_seq, int32_t* row_pos, const int32_t* token_to_seq,
                                    const int32_t* token_positions, const int32_t* seq_lens, int num_tokens,
                                    int num_reqs, vmc_stream_t stream) {
    if (num_tokens < 0 || num_reqs < 0) return VMC_EINVAL;
    if (num_tokens == 0) return VMC_OK;
    if (num_reqs == 0 || !row_seq || !row_pos || !token_to_seq || !token_positions || !seq_lens) return VMC_EINVAL;
    hipLaunchKernelGGL(batch_rows_kernel, dim3(1), dim3(kRowThreads), 0, reinterpret_cast<hipStream_t>(stream),
                       token_to_seq, token_positions, seq_lens, num_tokens, num_reqs, row_seq, row_pos);
    VMC_LAUNCH_CHECK();
    return VMC_OK;
}
