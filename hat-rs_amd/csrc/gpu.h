// The MI355X backend behind the reference's Backend interface.
//
// Reference seam: `trait Backend { fn name(); fn forward(h, w, input) }`
// (src/backend.rs:29-36) with `Gpu::new(&Weights)` (src/gpu.rs:372-386) and
// `Gpu::forward` (src/gpu.rs:759-803). Input is [3][h][w] in [0,1] (not
// mean-adjusted); output is [3][h*s][w*s] after denormalisation.
#pragma once
#include <map>
#include <string>
#include <vector>

#include "hip_rt.h"
#include "kargs.h"
#include "plan.h"
#include "weights.h"

namespace hat {

class Backend {
public:
    virtual ~Backend() {}
    virtual const char* name() const = 0;
    virtual void forward(int h, int w, const float* in, float* out) = 0;
};

struct DevLinear {
    float* w = nullptr;  // [N][Kp]
    float* b = nullptr;  // [N]
    // The same weights split into three bf16 parts for the split-bf16 kernels
    // (qkv: pack_linear_ws; projection: pack_linear_x, pack_linear_x180), or
    // null where the FP32 kernels run.
    unsigned short* wx = nullptr;
    int N = 0, K = 0, Kp = 0;
};

// The CAB of the compress-to-6 family, in the folded form (conv1 per-tap
// weights; conv2 and the channel attention as raw tensors for the gate kernel).
struct DevCab {
    unsigned short* w1 = nullptr;  // conv1 split for hat_cab_conv1* (CX_WPACK bf16)
    float* b1 = nullptr;  // [6]
    float* w2 = nullptr;  // [144][6][3][3]
    float* b2 = nullptr;  // [144]
    float* wa = nullptr;  // [sq][144]
    float* ba = nullptr;
    float* wb = nullptr;  // [144][sq]
    float* bb = nullptr;
};

// conv1 weight [6][144][3][3] -> 64 rows of 144 (row tap*6 + co holds
// w[co][:][tap], rows 54..63 zero), each weight as three bf16 parts in
// hat_cab_conv1's A-operand layout (CX_WPACK elements).
std::vector<unsigned short> pack_cab_conv1(const float* w);

// hat_mlpx's weights: the packed slices and b1 in fc1's row order.
struct DevMlpX {
    unsigned short* w = nullptr;  // C = 144: 24 weight chunks (pack_mlp_x); 180: 48 (pack_mlp_x180)
    unsigned short* wf = nullptr;  // the same in the fused tail's input order (pack_mlp_xf, pack_mlp_xf180)
    float* b1x = nullptr;          // fc1's bias in the fused tail's row order (pack_mlp_xf, pack_mlp_xf180)
    int C = 144;
};

struct DevConv {
    float* w = nullptr;  // [CIp/16][9][COp][16]
    float* b = nullptr;  // [COp]
    unsigned short* wu = nullptr;  // convs with a Winograd kernel: split U (pack_wino)
    int CI = 0, CIp = 0, CO = 0, COp = 0, r = 0;
};

// Host-side repacking (also used by the selftest and the op entry points).
std::vector<float> pack_linear(const float* w, int N, int K, int* Kp);
// [N][144] -> per 144-row slice, five weight chunks (one per 32-k step) of
// three bf16 planes [144][32] (k-groups swizzled as in pack_linear_ws): w =
// p0 + p1 + p2, each part the round-to-nearest bf16 of what the earlier ones
// leave; the fifth step (k = 128..143) packed, two parts per MFMA operand
// (split_half_step). The tails add the bias in fp32.
std::vector<unsigned short> pack_linear_x(const float* w, int N, int K);
// The same split for hat_gemmx_qkv's weight-stationary slices: per slice
// (144 rows at K = 144, 96 at 180) five or six chunks of three planes
// [rows][32], each row's 16-byte k-groups swizzled (ws_slot), WS_CHUNK
// elements apart. K = 144: the fifth step packed as in pack_linear_x, the bias
// not in the chunks (the kernel starts its accumulators from it); K = 180: the
// bias at k = 180.
std::vector<unsigned short> pack_linear_ws(const float* w, const float* bias, int N, int K);
// The C = 144 MLP (fc1 [288][144] + b1, fc2 [144][288]) for hat_mlpx: per
// third of the hidden layer eight weight chunks - five of fc1's 96 rows (b1
// as their column k = 144), then three of fc2 on those units - with fc1's
// rows in the order that leaves its output in fc2's operand layout
// (tailx.hip).
void pack_mlp_x(const float* w1, const float* b1, const float* w2, std::vector<unsigned short>* w);
// The same for the fused tails (hat_habx*), whose fc1 reads x' in the order a
// lane holds the projection's accumulators: input position k = 32 ks + 8 g + j
// of steps 0..3 is channel mlpx_fused_channel(k), step 4 (channels 128 ..
// 143) is packed as the K = 144 linears' last step, and b1 comes back in b1x
// (the thirds' permuted row order), added to fc1's output in fp32.
void pack_mlp_xf(const float* w1, const float* b1, const float* w2, std::vector<unsigned short>* w,
                 std::vector<float>* b1x);
int mlpx_fused_channel(int k);
// The C = 180 projection [180][180] for hat_projx180*: six chunks (one per
// 32-k step, k 180..191 zero) of three bf16 planes [192][32] (rows 180..191
// zero), k-groups swizzled as in pack_linear_ws, MX180_SLOT elements apart;
// the bias stays FP32 (added in the epilogue).
std::vector<unsigned short> pack_linear_x180(const float* w);
// The C = 180 MLP (fc1 [360][180] + b1, fc2 [180][360]) for hat_mlpx180: per
// part of MX180_HID hidden units six fc1 chunks (64 permuted rows, b1 as
// their column k = 180) then two fc2 chunks (192 rows), 48 chunks in all.
void pack_mlp_x180(const float* w1, const float* b1, const float* w2, std::vector<unsigned short>* w);
// The same for the fused C = 180 tails (hat_habx180*), whose fc1 reads x' in
// the order a lane holds the projection's accumulators: input position k =
// 32 ks + 8 g + j is channel mlpx180_fused_channel(k) (zero where that is -1),
// and b1 comes back in b1x (the parts' permuted row order), added to fc1's
// output in fp32.
void pack_mlp_xf180(const float* w1, const float* b1, const float* w2, std::vector<unsigned short>* w,
                    std::vector<float>* b1x);
int mlpx180_fused_channel(int k);
// Winograd U = G g G^T of a 3x3 conv [CO][CI][3][3] (formed in double), split
// into three bf16 parts in the layout convwino.hip streams:
// [32-channel chunk][point][16-channel tile][part][lane][8].
std::vector<unsigned short> pack_wino(const float* w, int CO, int CI, int r);
std::vector<float> pack_conv(const float* w, const float* b, int CO, int CI, int r,
                             std::vector<float>* bias_out, int* CIp, int* COp);
// A Winograd conv kernel (convwino.hip) over `tiles` 8 x 16 tiles in `ncb`
// column blocks (p.nblk set here). The persistent ones (convwino_persistent:
// the column-sum kernel) take a grid of at most one block a CU (or
// max_blocks), a multiple of ncb so that each block keeps its column block,
// each walking the virtual blocks blockIdx.x + i gridDim.x and fetching its
// next tile's first patch chunk under the current tile's epilogue; the others
// take one block a tile.
bool convwino_persistent(const std::string& name);
void launch_wino(hipStream_t s, const char* name, unsigned tiles, unsigned ncb, hatk::ConvArgs& p,
                 unsigned max_blocks = 0);

class GpuBackend : public Backend {
public:
    explicit GpuBackend(const Weights& wt);
    ~GpuBackend() override;
    const char* name() const override { return "gpu"; }
    void forward(int h, int w, const float* in, float* out) override;
    // Device-resident variant: d_in [3][h][w], d_out [3][h*s][w*s].
    void forward_device(int h, int w, const float* d_in, float* d_out);
    // The same pass with every per-plan buffer carved from the library's fixed
    // scratch array: no device memory is allocated. Throws if the plan does not
    // fit. Calls that overlap on one GPU share the array and race.
    void forward_noalloc(int h, int w, const float* d_in, float* d_out);
    // n images of one size, host [n][3][h][w] in, host [n][3][h*s][w*s] out:
    // up to kBatchSlots images in flight at once, each on its own stream with
    // its own per-plan buffers and pinned staging, so the kernels of several
    // small images fill the device together. Synchronous.
    void forward_batch(int n, int h, int w, const float* in, float* out);
    static constexpr int kBatchSlots = 4;
    // Bytes forward_noalloc needs at h x w.
    size_t noalloc_bytes(int h, int w) const;
    // Device bytes of the per-plan buffers a backend over `wt` allocates for an
    // h x w forward (gpu.rs:78-290 footprint_floats), computed without a device.
    static size_t plan_bytes(const Weights& wt, int h, int w, bool host_io);
    // Device bytes the weight upload of a backend over `wt` allocates (the
    // packed FP32 tensors and their split-bf16 copies), computed without a
    // device by running the upload's packers in a counting pass; cached in wt.
    static size_t device_weight_bytes(const Weights& wt);
    static bool cab_folded(const Weights& wt);
    // HAB.forward of one block (gpu.rs:469-520 `hab`) on a window-multiple
    // hp x wp plane: host x, out token-major [hp*wp][embed]; with the block's
    // shift and mask when it is odd. iters > 0: *ms = mean device time of the
    // block (its norm1 included) over that many further runs.
    void op_hab(int stage, int block, int hp, int wp, const float* x, float* out, int iters, float* ms);
    size_t acts_bytes() const { return acts_bytes_; }
    size_t weight_bytes() const { return weight_bytes_; }
    hipStream_t stream() const { return stream_; }
    const Weights& weights() const { return wt_; }

private:
    struct CountOnly {};
    GpuBackend(const Weights& wt, CountOnly);  // the counting pass: packs, uploads nothing
    void upload_all();
    const Weights& wt_;
    bool count_only_ = false;
    hipStream_t stream_ = nullptr;
    std::map<std::string, float*> raw_;
    std::map<std::string, DevLinear> lin_;
    std::map<std::string, DevConv> conv_;
    std::map<std::string, DevCab> cab_;
    std::map<std::string, DevMlpX> mlpx_;  // C = 144 MLPs (blocks and OCABs) for hat_mlpx
    bool cab_fold_ = false;  // the C = 144, 6-channel CAB runs folded
    std::vector<void*> owned_;
    size_t weight_bytes_ = 0;

    // The per-plan device buffers of one forward (Acts, gpu.rs:78-290). They
    // come from hipMalloc, once per input size (ensure_plan), or, for
    // forward_noalloc, from the library's fixed scratch array.
    struct Acts {
        float *x0 = nullptr, *body = nullptr, *xa = nullptr, *xb = nullptr, *xn = nullptr, *t1 = nullptr,
              *t2 = nullptr, *partial = nullptr, *red = nullptr, *gate = nullptr, *qkv = nullptr, *ao = nullptr,
              *hidden = nullptr, *head0 = nullptr, *head1 = nullptr, *din = nullptr, *dout = nullptr,
              *cab_part = nullptr, *w2g = nullptr, *w2gx = nullptr, *bias2 = nullptr;
    };
    // Each buffer of plan p and its size in floats (0: not used by this
    // network); host_io adds the staging buffers of the host-memory forward.
    static std::vector<std::pair<float**, size_t>> layout(const Weights& wt, const Plan& p, Acts& a,
                                                          bool host_io);

    Plan plan_;
    bool have_plan_ = false;
    std::vector<void*> acts_;
    size_t acts_bytes_ = 0;
    Acts a_;
    int t1_stride_ = 0, nblk_conv2_ = 0;

    // forward_batch's slots: a stream, a per-plan buffer set and pinned
    // staging each, kept for the last batch size.
    struct BatchSlot {
        hipStream_t s = nullptr;
        Acts a;
        float *hin = nullptr, *hout = nullptr;
        int img = -1;
    };
    std::vector<BatchSlot> batch_;
    Plan batch_plan_;
    std::vector<void*> batch_dev_;
    void free_batch();

    // Backend::forward's host staging, kept for the plan: pinned input and
    // output buffers; the stream that downloads the output bands, an event per
    // band on each stream (computed, downloaded).
    float *stage_in_ = nullptr, *stage_out_ = nullptr;
    size_t stage_in_n_ = 0, stage_out_n_ = 0;
    hipStream_t copy_stream_ = nullptr;
    std::vector<hipEvent_t> band_ev_, copy_ev_;
    void free_stage();

    float* upload(const float* src, size_t n);
    void* upload_bytes(const void* src, size_t bytes);
    void upload_raw(const std::string& name);
    void upload_linear(const std::string& name);
    void upload_conv(const std::string& name, int r = 0);
    void upload_mlpx(const std::string& name);
    void ensure_plan(int h, int w);
    void free_plan();
    // With bands: the output's row bands [y0, y1) in the order they are
    // written, band_ev_[k] recorded on the stream after band k (the
    // host-memory forward downloads each while later ones compute).
    void run_forward(int h, int w, const float* d_in, float* d_out,
                     std::vector<std::pair<int, int>>* bands = nullptr);
    bool head_bands_fit(const DevConv& up, const DevConv& last, int hh, int ww, int feat) const;

    void layernorm(const float* x, float* y, const std::string& prefix, long rows);
    void gemm(const DevLinear& L, const float* a, int lda, long M, float* out, int ldo, int epi,
              const float* res = nullptr, const float* aux = nullptr, const float* gate = nullptr,
              float* xn = nullptr, const std::string& norm = "");
    void conv(const DevConv& C, const float* in, int cin_stride, int H, int W, float* out,
              int co_stride, int epi, int act, const float* res = nullptr, float* partial = nullptr,
              int crop_h = 0, int crop_w = 0, int band_r0 = 0, int band_r1 = -1);
    void attention(const std::string& table, bool oca, int shift, const hatk::CabGateArgs* gate = nullptr,
                   const hatk::SeArgs* se = nullptr);
    void mlp(const std::string& prefix, float* x, int epi, const std::string& norm);
    void hab(int stage, int block, float* x_in, float* x_out, const std::string& next_norm);
    void ocab(int stage, float* x);
};

// Isolated ops on host buffers (cfg2 / cfg3 of the benchmark plan). Each
// uploads, runs `warmup + iters` times, downloads, and reports the mean device
// time per run (HIP events on the op's stream) in *ms when ms is non-null.
void op_swmsa(const float* x, float* out, int hp, int wp, int c, int heads, int shift,
              const float* qkv_w, const float* qkv_b, const float* proj_w, const float* proj_b,
              const float* table, int iters, float* ms, float* attn_ms);
void op_ocab(const float* x, float* out, int hp, int wp, int c, int heads, int mlp_ratio,
             const float* n1w, const float* n1b, const float* qkv_w, const float* qkv_b,
             const float* proj_w, const float* proj_b, const float* table, const float* n2w,
             const float* n2b, const float* fc1_w, const float* fc1_b, const float* fc2_w,
             const float* fc2_b, int iters, float* ms, float* attn_ms);

// Selftest: every kernel against a host twin. Prints "  ok  <name>" per pass.
int gpu_selftest(std::string* err);

}  // namespace hat
