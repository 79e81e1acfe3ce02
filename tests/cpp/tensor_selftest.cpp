// Self-test of the C++ tensor layer (cudasep::Tensor, tensor_tile::, mbr_tile::) on a GPU.
//
//   tensor_selftest unit        Tensor / allocator semantics against expectations computed
//                               here on the host; prints one line per check, exit status =
//                               number of failures.
//   tensor_selftest ops <dir>   runs the mbr_tile ops on the inputs that tests/test_cpp_layer.py
//                               wrote to <dir> and writes their outputs there for comparison
//                               with the oracle.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <iostream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/mbrt.h"
#include "hip_context.h"
#include "mbr_tile.h"
#include "stft_tile.h"
#include "chunk_tile.h"
#include "weights.h"
#include "memory_pool.h"
#include "tensor.h"

using cudasep::DType;
using cudasep::Tensor;

namespace {

int g_fail = 0;

void check(bool ok, const std::string& what) {
    std::cout << (ok ? "PASS " : "FAIL ") << what << std::endl;
    if (!ok) ++g_fail;
}

bool same(const std::vector<float>& a, const std::vector<float>& b) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); ++i)
        if (!(a[i] == b[i])) return false;
    return true;
}

template <class F>
void expect_throw(F f, const std::string& needle, const std::string& what) {
    try {
        f();
    } catch (const std::exception& e) {
        const bool ok = std::string(e.what()).find(needle) != std::string::npos;
        if (!ok) std::cout << "  message: " << e.what() << std::endl;
        check(ok, what);
        return;
    }
    check(false, what + " (no exception)");
}

Tensor host_f32(const std::vector<float>& v, std::vector<int64_t> shape) { return Tensor::from_cpu_f32(v.data(), shape); }

std::vector<float> iota_f(int n, float start = 0.0f) {
    std::vector<float> v(n);
    for (int i = 0; i < n; ++i) v[i] = start + (float)i;
    return v;
}

// Host reference of a strided read: out[i] = src[sum_d coord_d(i) * stride_d]
std::vector<float> gather_strided(const std::vector<float>& src, const std::vector<int64_t>& shape,
                                  const std::vector<int64_t>& strides, int64_t offset = 0) {
    int64_t n = 1;
    for (int64_t s : shape) n *= s;
    std::vector<float> out(n);
    for (int64_t i = 0; i < n; ++i) {
        int64_t r = i, off = offset;
        for (int d = (int)shape.size() - 1; d >= 0; --d) {
            off += (r % shape[d]) * strides[d];
            r /= shape[d];
        }
        out[i] = src[off];
    }
    return out;
}

void unit() {
    // factories
    check(same(Tensor::zeros({5}).to_cpu_f32(), std::vector<float>(5, 0.0f)), "zeros");
    check(same(Tensor::ones({2, 3}).to_cpu_f32(), std::vector<float>(6, 1.0f)), "ones");
    check(same(Tensor::full({4}, 2.5f, DType::Float16).to_cpu_f32(), std::vector<float>(4, 2.5f)), "full f16");
    check(same(Tensor::arange(3, 10).to_cpu_f32(), iota_f(7, 3)), "arange f32");
    check(same(Tensor::arange(-2, 3, DType::Int64).to_cpu_f32(), iota_f(5, -2)), "arange i64");
    check(Tensor::arange(5, 5).numel() == 0 && Tensor::arange(5, 5).ndim() == 0, "arange empty range -> Tensor()");
    expect_throw([] { Tensor::arange(0, 4, DType::BFloat16); }, "arange: unsupported BF16 dtype", "arange bf16 throws");

    // views
    const std::vector<float> base = iota_f(24);
    Tensor x = host_f32(base, {2, 3, 4});
    check(x.is_contiguous() && x.strides() == std::vector<int64_t>({12, 4, 1}), "contiguous strides");
    Tensor p = x.permute({2, 0, 1});
    check(!p.is_contiguous() && p.shape() == std::vector<int64_t>({4, 2, 3}) && p.data_ptr() == x.data_ptr(),
          "permute is a view");
    check(same(p.contiguous().to_cpu_f32(), gather_strided(base, {4, 2, 3}, {1, 12, 4})), "permute + contiguous");
    check(same(x.transpose(-1, 0).contiguous().to_cpu_f32(), gather_strided(base, {4, 3, 2}, {1, 4, 12})),
          "transpose negative dims");
    Tensor sl = x.slice(1, 1, 3);
    check(sl.shape() == std::vector<int64_t>({2, 2, 4}) && !sl.is_contiguous(), "slice shape");
    check(same(sl.contiguous().to_cpu_f32(), gather_strided(base, {2, 2, 4}, {12, 4, 1}, 4)), "slice values");
    check(x.slice(2, -1, 100).contiguous().to_cpu_f32() == gather_strided(base, {2, 3, 1}, {12, 4, 1}, 3),
          "slice negative start, clamped end");
    check(x.slice(0, 2, 1).numel() == 0, "empty slice");
    check(same(x.reshape({4, -1}).to_cpu_f32(), base) && x.reshape({4, -1}).shape() == std::vector<int64_t>({4, 6}),
          "reshape -1");
    check(same(p.reshape({24}).to_cpu_f32(), gather_strided(base, {4, 2, 3}, {1, 12, 4})),
          "reshape of a non-contiguous view copies");
    expect_throw([&] { x.reshape({5, 5}); }, "reshape: incompatible sizes 24 vs 25", "reshape size error");
    check(x.unsqueeze(0).shape() == std::vector<int64_t>({1, 2, 3, 4}) &&
              x.unsqueeze(-1).shape() == std::vector<int64_t>({2, 3, 4, 1}),
          "unsqueeze");
    check(x.unsqueeze(1).squeeze(1).shape() == x.shape(), "squeeze");
    expect_throw([&] { x.squeeze(0); }, "squeeze: dimension is not 1", "squeeze error");
    Tensor col = host_f32({1, 2, 3}, {3, 1});
    Tensor ex = col.expand({2, 3, 4});
    check(ex.strides() == std::vector<int64_t>({0, 1, 0}) && ex.numel() == 24, "expand strides");
    check(same(ex.contiguous().to_cpu_f32(), gather_strided({1, 2, 3}, {2, 3, 4}, {0, 1, 0})), "expand values");
    expect_throw([&] { col.expand({2, 4}); }, "expand: incompatible shape", "expand error");
    check(Tensor::empty({1, 3, 1}).is_contiguous(), "size-1 dims ignored by is_contiguous");

    // dtype conversion
    Tensor small = host_f32({-3, -1.5f, 0, 2, 255, 1e-3f}, {6});
    std::vector<float> rt = small.to_bf16().to_f32().to_cpu_f32();
    check(rt[0] == -3 && rt[1] == -1.5f && rt[3] == 2 && rt[4] == 255, "f32 -> bf16 -> f32");
    check(small.to_dtype(DType::Float32).data_ptr() == small.data_ptr(), "to_dtype same dtype is a view");
    expect_throw([&] { small.to_f16().to_bf16(); }, "to_dtype: unsupported conversion", "f16 -> bf16 rejected");
    check(same(host_f32({1.9f, -1.9f}, {2}).to_dtype(DType::Int64).to_cpu_f32(), {1, -1}), "f32 -> i64 truncates");

    // element-wise
    Tensor a = host_f32(iota_f(6), {2, 3}), b = host_f32(iota_f(6, 10), {2, 3});
    check(same((a + b).to_cpu_f32(), {10, 12, 14, 16, 18, 20}), "add same shape");
    check(same((b - a).to_cpu_f32(), std::vector<float>(6, 10)), "sub");
    check(same((a * b).to_cpu_f32(), {0, 11, 24, 39, 56, 75}), "mul");
    Tensor r = host_f32({1, 2, 3}, {3});
    check(same((a + r).to_cpu_f32(), {1, 3, 5, 4, 6, 8}), "broadcast row");
    Tensor c2 = host_f32({10, 20}, {2, 1});
    check(same((a * c2).to_cpu_f32(), {0, 10, 20, 60, 80, 100}), "broadcast column");
    check(same((a.transpose(0, 1) + r.unsqueeze(1)).to_cpu_f32(), {1, 4, 3, 6, 5, 8}), "broadcast strided operand");
    check(same((-a).to_cpu_f32(), {-0.f, -1, -2, -3, -4, -5}), "negate");
    check(same((a > 2.5f).to_cpu_f32(), {0, 0, 0, 1, 1, 1}), "greater_than");
    expect_throw([&] { (void)(a + a.to_f16()); }, "dtype mismatch", "binary dtype mismatch");
    Tensor acc = a.clone();
    acc.add_(r);
    check(same(acc.to_cpu_f32(), {1, 3, 5, 4, 6, 8}), "add_ broadcast in place");
    acc.mul_(acc);
    check(same(acc.to_cpu_f32(), {1, 9, 25, 16, 36, 64}), "mul_ same shape in place");
    Tensor tv = a.clone().transpose(0, 1);
    expect_throw([&] { tv.add_(r.slice(0, 0, 2)); }, "must be contiguous", "in-place onto a non-contiguous view");
    Tensor s = a.clone();
    s.add_scalar_(1.5f).mul_scalar_(2.0f).clamp_(4.0f, 10.0f);
    check(same(s.to_cpu_f32(), {4, 5, 7, 9, 10, 10}), "add_scalar_ / mul_scalar_ / clamp_");
    s.fill_(-7.0f);
    check(same(s.to_cpu_f32(), std::vector<float>(6, -7)), "fill_");
    expect_throw([&] { Tensor t = a.to_bf16(); t.add_scalar_(1.0f); }, "add_scalar_: unsupported dtype",
                 "add_scalar_ bf16 rejected");

    // reductions
    check(same(x.sum(2).to_cpu_f32(), {6, 22, 38, 54, 70, 86}), "sum last dim");
    check(same(x.sum(0).to_cpu_f32(), {12, 14, 16, 18, 20, 22, 24, 26, 28, 30, 32, 34}), "sum dim 0");
    check(x.sum(1, true).shape() == std::vector<int64_t>({2, 1, 4}), "sum keepdim shape");
    check(same(x.sum(1).to_cpu_f32(), {12, 15, 18, 21, 48, 51, 54, 57}), "sum middle dim");
    check(same(x.max(-1).to_cpu_f32(), {3, 7, 11, 15, 19, 23}), "max last dim");
    check(same(x.mean(2).to_cpu_f32(), {1.5f, 5.5f, 9.5f, 13.5f, 17.5f, 21.5f}), "mean");
    check(same(x.to_bf16().sum(2).to_cpu_f32(), {6, 22, 38, 54, 70, 86}), "sum of bf16 converts first");

    // cat / stack / split / unbind
    Tensor u = host_f32({1, 2, 3, 4}, {2, 2}), v = host_f32({5, 6}, {2, 1});
    check(same(Tensor::cat({u, v}, 1).to_cpu_f32(), {1, 2, 5, 3, 4, 6}), "cat dim 1");
    check(same(Tensor::cat({u, u.slice(0, 1, 2)}, 0).to_cpu_f32(), {1, 2, 3, 4, 3, 4}), "cat dim 0");
    check(Tensor::stack({u, u}, 0).shape() == std::vector<int64_t>({2, 2, 2}), "stack shape");
    check(same(Tensor::stack({u, u}, 2).to_cpu_f32(), {1, 1, 2, 2, 3, 3, 4, 4}), "stack last dim");
    expect_throw([&] { Tensor::cat({u, u.to_f16()}, 0); }, "cat: dtype mismatch", "cat dtype mismatch");
    auto parts = x.split(2, {1, 3});
    check(parts.size() == 2 && parts[1].shape() == std::vector<int64_t>({2, 3, 3}) &&
              same(parts[0].contiguous().to_cpu_f32(), {0, 4, 8, 12, 16, 20}),
          "split");
    auto ub = x.unbind(0);
    check(ub.size() == 2 && ub[1].shape() == std::vector<int64_t>({3, 4}) && same(ub[1].to_cpu_f32(), iota_f(12, 12)),
          "unbind");

    // padding
    Tensor row = host_f32({1, 2, 3, 4}, {1, 4});
    check(same(row.pad({2, 1}, -1.0f).to_cpu_f32(), {-1, -1, 1, 2, 3, 4, -1}), "pad const");
    check(same(row.pad_reflect({2, 2}).to_cpu_f32(), {3, 2, 1, 2, 3, 4, 3, 2}), "pad reflect");
    check(row.pad({1, 1, 1, 0}).shape() == std::vector<int64_t>({2, 6}), "pad two dims shape");
    check(same(x.slice(2, 1, 3).pad({1, 0}).to_cpu_f32(),
               {0, 1, 2, 0, 5, 6, 0, 9, 10, 0, 13, 14, 0, 17, 18, 0, 21, 22}),
          "pad of a strided view");

    // index_select
    const int64_t idx_h[3] = {2, 0, 2};
    Tensor idx = Tensor::from_cpu_i64(idx_h, {3});
    check(same(x.index_select(1, idx).to_cpu_f32(),
               {8, 9, 10, 11, 0, 1, 2, 3, 8, 9, 10, 11, 20, 21, 22, 23, 12, 13, 14, 15, 20, 21, 22, 23}),
          "index_select dim 1");
    expect_throw([&] { x.index_select(0, idx.to_f32()); }, "indices must be Int64", "index_select dtype");

    // copies
    Tensor cl = p.clone();
    check(cl.is_contiguous() && same(cl.to_cpu_f32(), p.contiguous().to_cpu_f32()), "clone of a view");
    Tensor dst = Tensor::empty({4, 2, 3});
    dst.copy_from(p);
    check(same(dst.to_cpu_f32(), cl.to_cpu_f32()), "copy_from a strided view");
    expect_throw([&] { dst.copy_from(u); }, "copy_from: size mismatch", "copy_from size");
    std::vector<float> host(6);
    a.copy_to_cpu(host.data(), 24);
    check(same(host, iota_f(6)), "copy_to_cpu");
    check(same(Tensor::from_cpu_i64(idx_h, {3}).to_cpu_f32(), {2, 0, 2}), "i64 to_cpu_f32");
    check(x.size(-1) == 4 && x.shape_str() == "(2, 3, 4)", "size / shape_str");
    expect_throw([&] { x.size(3); }, "dim out of range", "size out of range");

    // allocator
    auto& pool = cudasep::HipMemoryPool::instance();
    check(pool.round_up(1) == 512 && pool.round_up(513) == 1024 && pool.round_up((1 << 20) + 1) == (2u << 20) &&
              pool.round_up(5u << 20) == (6u << 20),
          "allocator rounding");
    const auto before = pool.get_stats();
    { Tensor t1 = Tensor::empty({1 << 20}); }
    { Tensor t2 = Tensor::empty({(1 << 20) - 7}); }
    const auto after = pool.get_stats();
    check(after.cache_hits >= before.cache_hits + 1, "freed block is reused");
    pool.trim_cached_memory();
    check(pool.get_stats().cached_bytes == 0, "trim releases the cache");

    // set_stream: the work queued on the old stream is done before any work on the new
    // one, so a block freed under pending work cannot be reused while that work runs
    {
        auto& ctx = cudasep::HipContext::instance();
        hipStream_t s1 = nullptr, s2 = nullptr;
        HIP_CHECK(hipStreamCreate(&s1));
        HIP_CHECK(hipStreamCreate(&s2));
        ctx.set_stream(s1);
        Tensor big = Tensor::empty({1 << 26});
        big.fill_(1.0f);
        for (int i = 0; i < 8; ++i) big.add_(big);  // queued work on s1
        { Tensor freed = big + big; }  // its block goes back to the cache with work pending on s1
        ctx.set_stream(s2);
        check(hipStreamQuery(s1) == hipSuccess, "set_stream waits for the previous stream");
        check(same(big.slice(0, 0, 4).to_cpu_f32(), std::vector<float>(4, 256.0f)), "work of the old stream kept");
        ctx.set_stream(nullptr);
        HIP_CHECK(hipStreamDestroy(s1));
        HIP_CHECK(hipStreamDestroy(s2));
    }

    // set_stream while the current stream is being captured into a graph: it must not
    // synchronize (that would invalidate the capture); the new stream joins the capture,
    // and switching back joins it again, so the capture ends cleanly.  The graph is then
    // replayed several times with eager work in between, each replay checked.
    {
        auto& ctx = cudasep::HipContext::instance();
        hipStream_t s1 = nullptr, s2 = nullptr;
        HIP_CHECK(hipStreamCreate(&s1));
        HIP_CHECK(hipStreamCreate(&s2));
        ctx.set_stream(s1);
        Tensor y = Tensor::empty({4096});  // allocated before the capture
        y.fill_(0.0f);
        ctx.synchronize();
        HIP_CHECK(hipStreamBeginCapture(s1, hipStreamCaptureModeRelaxed));
        bool switched = true;
        try {
            y.fill_(2.0f);     // captured on s1
            ctx.set_stream(s2);
            y.add_(y);         // captured on s2, after the fill
            ctx.set_stream(s1);
            y.mul_scalar_(3.0f);  // captured on s1, after the add
        } catch (const std::exception& e) {
            std::cout << "  message: " << e.what() << std::endl;
            switched = false;
            ctx.set_stream(s1);
        }
        hipGraph_t graph = nullptr;
        const hipError_t end = hipStreamEndCapture(s1, &graph);
        check(switched && end == hipSuccess && graph != nullptr, "set_stream inside a capture keeps the capture valid");
        if (end == hipSuccess && graph != nullptr) {
            hipGraphExec_t exec = nullptr;
            HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
            bool all = true;
            for (int rep = 0; rep < 3; ++rep) {
                y.fill_(-1.0f);  // eager work between replays
                ctx.synchronize();
                HIP_CHECK(hipGraphLaunch(exec, s1));
                HIP_CHECK(hipStreamSynchronize(s1));
                all = all && same(y.to_cpu_f32(), std::vector<float>(4096, 12.0f));
            }
            check(all, "graph captured across set_stream replays (2 + 2) * 3 = 12, three times");
            HIP_CHECK(hipGraphExecDestroy(exec));
            HIP_CHECK(hipGraphDestroy(graph));
        }
        ctx.set_stream(nullptr);
        HIP_CHECK(hipStreamDestroy(s1));
        HIP_CHECK(hipStreamDestroy(s2));
    }
}

// ---- ops mode: raw little-endian inputs/outputs named in <dir>/manifest.txt -------------

struct Dir {
    std::string path;
    std::map<std::string, Tensor> in;

    Tensor load(const std::string& name, DType dt, const std::vector<int64_t>& shape) {
        Tensor t = Tensor::empty(shape, dt);
        std::ifstream f(path + "/" + name + ".bin", std::ios::binary);
        std::vector<char> buf((size_t)t.numel() * cudasep::dtype_size(dt));
        f.read(buf.data(), (std::streamsize)buf.size());
        if (!f) throw std::runtime_error("cannot read input " + name);
        t.copy_from_cpu(buf.data(), buf.size());
        return t;
    }
    void save(const std::string& name, const Tensor& t) {
        Tensor c = t.contiguous();
        std::vector<char> buf((size_t)c.numel() * cudasep::dtype_size(c.dtype()));
        c.copy_to_cpu(buf.data(), buf.size());
        std::ofstream f(path + "/" + name + ".out", std::ios::binary);
        f.write(buf.data(), (std::streamsize)buf.size());
        std::ofstream m(path + "/" + name + ".meta");
        m << (int)c.dtype();
        for (int64_t s : c.shape()) m << " " << s;
        m << "\n";
    }
};

// manifest lines: <name> <dtype code> <ndim> <dims...>
void ops(const std::string& path) {
    Dir d{path, {}};
    std::ifstream man(path + "/manifest.txt");
    std::string line;
    while (std::getline(man, line)) {
        std::istringstream ls(line);
        std::string name;
        int dt, nd;
        if (!(ls >> name >> dt >> nd)) continue;
        std::vector<int64_t> shape(nd);
        for (int i = 0; i < nd; ++i) ls >> shape[i];
        d.in[name] = d.load(name, (DType)dt, shape);
    }
    namespace M = cudasep::mbr_tile;
    auto& I = d.in;
    const float scale = std::sqrt(384.0f);
    cudasep::g_quantize_bf16 = false;
    d.save("rms_norm", M::rms_norm(I["x"], I["gamma"], scale));
    Tensor sum, normed;
    const bool fused = M::try_residual_add_rms_norm(I["x"], I["res"], I["gamma"], scale, sum, normed);
    check(fused, "try_residual_add_rms_norm fuses f32 rows of 384");
    d.save("resid_sum", sum);
    d.save("resid_normed", normed);
    d.save("softmax", M::softmax_last_dim(I["scores"], 0.125f, DType::Float32));
    Tensor sm_inplace = I["scores"].clone();
    M::softmax_last_dim_(sm_inplace, 0.125f);
    d.save("softmax_inplace", sm_inplace);
    d.save("gelu_ref", M::add_bias_activation(I["h"], &I["bias"], M::Activation::GeluRef, DType::BFloat16));
    d.save("gather", M::gather_freqs_fold_complex(I["stft"], I["freq_indices"]));
    d.save("merge", M::apply_mask_and_scatter(I["stft"], {I["mask0"], I["mask1"]}, I["freq_indices"], I["csr_off"],
                                              I["csr_ind"], I["counts"], I["stft"].size(0), 2, I["stft"].size(1),
                                              I["freq_indices"].numel(), I["stft"].size(2), 2));
    d.save("merge_rebuilt_csr",
           M::apply_mask_and_scatter(I["stft"], {I["mask0"]}, I["freq_indices"], Tensor(), Tensor(), I["counts"],
                                     I["stft"].size(0), 1, I["stft"].size(1), I["freq_indices"].numel(),
                                     I["stft"].size(2), 2));
    Tensor spec = I["stft"].clone().reshape({I["stft"].size(0) * 2, I["stft"].size(1) / 2, I["stft"].size(2), 2});
    M::zero_dc(spec);
    d.save("zero_dc", spec);
    // bf16 mode: policies switch the outputs to bf16
    cudasep::g_quantize_bf16 = true;
    d.save("glu_bf16", M::glu_last_dim(I["g"]));
    d.save("gates_merge", M::apply_gates_and_merge_heads(I["attn"], I["gates"], 8, 64));
    d.save("gate_logits_merge", M::apply_gate_logits_and_merge_heads(I["attn"], I["logits"], 8, 64));
    Tensor q = I["q"].clone(), k = I["k"].clone();
    M::apply_rotary_time_split_contig_inplace(q, k, I["cos"], I["sin"]);
    d.save("rot_q", q);
    d.save("rot_k", k);
    {
        Tensor qa = I["q"].permute({0, 2, 1, 3}).contiguous();  // [B, H, N, D]
        Tensor ka = I["k"].permute({0, 2, 1, 3}).contiguous();
        d.save("attention", M::scaled_dot_product_attention(qa, ka, ka, 0.0f));
        // the split-contig forms read [B, N, H, D] in place; the q-rotary one rotates q itself
        d.save("attention_split_contig", M::scaled_dot_product_attention_time_split_contig(I["q"], I["k"], I["k"], 0.0f));
        d.save("attention_split_contig_qrot",
               M::scaled_dot_product_attention_time_split_contig_q_rotary(I["q"], k, k, I["cos"], I["sin"], 0.0f));
        Tensor rqa = q.permute({0, 2, 1, 3}).contiguous(), rka = k.permute({0, 2, 1, 3}).contiguous();
        d.save("attention_rotated", M::scaled_dot_product_attention(rqa, rka, rka, 0.0f));
    }
    Tensor sq, sk, sv;
    M::split_qkv_heads_rotary(I["qkv"], 8, 64, I["cos"], I["sin"], sq, sk, sv);
    d.save("split_q", sq);
    d.save("split_k", sk);
    d.save("split_v", sv);
    {
        // CUDASEP_FULL_BF16_ARITH_EXPERIMENTS under bf16: these ops round their
        // intermediates to bf16 while they run and leave the thread's C-ABI flags as found
        setenv("CUDASEP_FULL_BF16_ARITH_EXPERIMENTS", "1", 1);
        d.save("full_rms_norm", M::rms_norm(I["x"], I["gamma"], scale));
        d.save("full_glu", M::glu_last_dim(I["g"]));
        d.save("full_softmax", M::softmax_last_dim(I["scores"].to_bf16(), 0.125f, DType::BFloat16));
        d.save("full_gate_logits_merge", M::apply_gate_logits_and_merge_heads(I["attn"], I["logits"], 8, 64));
        d.save("full_merge", M::apply_mask_and_scatter(I["stft"], {I["mask0"], I["mask1"]}, I["freq_indices"],
                                                       I["csr_off"], I["csr_ind"], I["counts"], I["stft"].size(0), 2,
                                                       I["stft"].size(1), I["freq_indices"].numel(),
                                                       I["stft"].size(2), 2));
        unsetenv("CUDASEP_FULL_BF16_ARITH_EXPERIMENTS");
        if (mbrt_get_arith_flags() != 0) throw std::runtime_error("mbr_tile left the bf16-intermediates flag set");
    }
    {
        namespace S = cudasep::stft_tile;
        const Tensor hann = S::hann_window(2048);
        d.save("hann", hann);
        const Tensor spec = S::stft(I["signal"], 2048, 441, 2048, hann);  // [2, 5000] -> [2, 1025, 12, 2]
        d.save("stft", spec);
        d.save("istft", S::istft(spec, 2048, 441, 2048, hann, 5000));
        d.save("istft_bf16", S::istft(spec.to_bf16(), 2048, 441, 2048, hann));
        bool threw = false;
        try {
            S::stft(I["signal"], 1024, 441, 1024, hann);
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()) == "custom STFT only supports n_fft=2048, win_length=2048";
        }
        if (!threw) throw std::runtime_error("stft_tile::stft accepted n_fft=1024");
    }
    {
        namespace K = cudasep::chunk_tile;
        auto identity = [](const Tensor& x) { return x.clone(); };
        auto two_stems = [](const Tensor& x) {  // [G, C, n] -> [G, 2, C, n] = (2x, -x)
            Tensor a = x.clone(), b = x.clone();
            a.mul_scalar_(2.0f);
            b.mul_scalar_(-1.0f);
            return Tensor::stack({a, b}, 1);
        };
        std::vector<std::string> log;
        auto logger = [&log](const std::string& m) { log.push_back(m); };
        // the model sees the index of the first chunk of its call as the time-attention
        // chunk context, and the context is unset again after the pass
        std::vector<int> seen;
        auto identity_ctx = [&seen](const Tensor& x) {
            seen.push_back(cudasep::mbr_tile::time_attention_context_chunk());
            return x.clone();
        };
        d.save("chunk_a_b1", K::process_chunked(I["audio_a"], 4000, 3000, 1, identity));
        d.save("chunk_a_b4", K::process_chunked(I["audio_a"], 4000, 3000, 4, identity_ctx, logger));
        d.save("chunk_b_2stem", K::process_chunked(I["audio_b"], 4000, 3200, 2, two_stems));
        d.save("chunk_c_short", K::process_chunked(I["audio_c"], 4000, 3000, 3, identity));
        if (log.size() != seen.size() + 1 || log.front().rfind("chunked pass: ", 0) != 0 ||
            log.back().find(" chunk(s) merged") == std::string::npos)
            throw std::runtime_error("chunk_tile::process_chunked: unexpected log lines");
        bool ctx_ok = !seen.empty() && cudasep::mbr_tile::time_attention_context_chunk() == -1;
        for (size_t i = 0; i < seen.size(); ++i) ctx_ok = ctx_ok && seen[i] == 4 * (int)i;
        if (!ctx_ok) throw std::runtime_error("chunk_tile::process_chunked: unexpected attention chunk context");
        cudasep::mbr_tile::set_time_attention_context_depth(3);
        if (cudasep::mbr_tile::time_attention_context_depth() != 3)
            throw std::runtime_error("mbr_tile::set_time_attention_context_depth not kept");
        cudasep::mbr_tile::set_time_attention_context_depth(-1);
    }
    cudasep::g_quantize_bf16 = false;
    cudasep::HipContext::instance().synchronize();
}

// ---- csm mode: .csm loader, JSON, band tables --------------------------------------------

void json_dump(std::ostream& o, const cudasep::JsonValue& v) {
    using J = cudasep::JsonValue;
    switch (v.type()) {
        case J::Null: o << "null"; break;
        case J::Bool: o << (v.as_bool() ? "true" : "false"); break;
        case J::Number: {
            char b[64];
            std::snprintf(b, sizeof b, "%.17g", v.as_number());
            o << b;
            break;
        }
        case J::String: {
            o << '"';
            for (unsigned char c : v.as_string()) {
                if (c == '"' || c == '\\') o << '\\' << c;
                else if (c < 0x20) {
                    char b[8];
                    std::snprintf(b, sizeof b, "\\u%04x", c);
                    o << b;
                } else o << c;
            }
            o << '"';
            break;
        }
        case J::Array:
            o << '[';
            for (size_t i = 0; i < v.size(); ++i) {
                if (i) o << ',';
                json_dump(o, v[i]);
            }
            o << ']';
            break;
        case J::Object: {
            o << '{';
            bool first = true;
            for (const auto& k : v.keys()) {
                if (!first) o << ',';
                first = false;
                json_dump(o, J::make_string(k));
                o << ':';
                json_dump(o, v[k]);
            }
            o << '}';
            break;
        }
    }
}

void csm(const std::string& path) {
    using cudasep::ModelWeights;
    Dir d{path, {}};
    // JSON cases, one per line: canonical dump or "ERR <message>"
    {
        std::ifstream in(path + "/json_cases.txt");
        std::ofstream out(path + "/json_out.txt");
        std::string line;
        while (std::getline(in, line)) {
            try {
                json_dump(out, cudasep::JsonValue::parse(line));
            } catch (const std::exception& e) {
                out << "ERR " << e.what();
            }
            out << "\n";
        }
    }
    // a model file: tensors in sorted-name order, the config, band tables, bf16 conversion
    ModelWeights w = ModelWeights::load(path + "/model.csm");
    {
        std::ofstream names(path + "/names.txt");
        int i = 0;
        for (const auto& n : w.tensor_names()) {
            names << n << "\n";
            d.save("t" + std::to_string(i++), w.get(n));
        }
        std::ofstream cfg(path + "/config_out.txt");
        json_dump(cfg, w.config());
        cfg << "\n" << w.config().get_int("num_bands", -1) << " " << w.config().get_int("missing", 7) << " "
            << w.config().get_float("stft_hop_length", -1.f) << " " << w.config().get_bool("stereo", false) << " "
            << w.config().get_string("model_type", "none") << "\n";
        check(w.arena_bytes() % 256 == 0, "arena is a multiple of 256 bytes");
        bool threw = false;
        try {
            (void)w.get("no.such.tensor");
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()) == "ModelWeights: tensor not found: no.such.tensor";
        }
        check(threw, "get() of a missing tensor throws the reference's message");
    }
    if (w.has("__precomputed__.freq_indices")) {
        const auto& c = w.config();
        cudasep::MelBandTables t = cudasep::load_mel_band_tables(w, c.get_int("num_bands", 60),
                                                                 c.get_int("stft_n_fft", 2048), c.get_bool("stereo", true));
        d.save("band_offsets", t.freq_band_offsets);
        d.save("band_indices", t.freq_band_indices);
        d.save("band_counts", t.num_bands_per_freq);
        std::ofstream o(path + "/band_dims.txt");
        o << t.max_bands_per_freq;
        for (int64_t x : t.band_freq_dims) o << " " << x;
        o << "\n";
    }
    w.convert_linear_weights_to_bf16();
    {
        int i = 0;
        for (const auto& n : w.tensor_names()) d.save("c" + std::to_string(i++), w.get(n));
    }
    // malformed files: each load must throw; the message is recorded
    std::ofstream errs(path + "/errors.txt");
    for (const char* bad : {"bad_magic", "bad_version", "truncated", "bad_dtype", "missing", "huge_bytes", "huge_numel"}) {
        try {
            (void)ModelWeights::load(path + "/" + bad + ".csm");
            errs << bad << " LOADED\n";
        } catch (const std::exception& e) {
            errs << bad << " " << e.what() << "\n";
        }
    }
    cudasep::HipContext::instance().synchronize();
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "unit";
    try {
        if (mode == "unit") unit();
        else if (mode == "ops" && argc > 2) ops(argv[2]);
        else if (mode == "csm" && argc > 2) csm(argv[2]);
        else {
            std::cerr << "usage: tensor_selftest unit | ops <dir> | csm <dir>" << std::endl;
            return 2;
        }
    } catch (const std::exception& e) {
        std::cout << "FAIL exception: " << e.what() << std::endl;
        return 100;
    }
    std::cout << (g_fail ? "FAILED " : "OK ") << g_fail << std::endl;
    return g_fail;
}
