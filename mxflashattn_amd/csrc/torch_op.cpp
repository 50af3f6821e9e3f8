// Host-side torch operator in front of the C ABI (include/mxfa_mi355x.h): the
// hot decode call and the vLLM-form page append without Python's
// per-argument marshalling.
//
// decode(q, k_cache, v_cache, block_table, cache_seqlens, scale, out,
//        num_splits, seqlen_add) takes the common call (one query
// token per sequence, caches of q's 16-bit type, int32 table and lengths,
// every tensor on the current GPU with layouts the kernels read in place),
// launches it on torch's current HIP stream and returns the output.
// num_splits None is mxfa_split_heuristic's choice. For any
// other call it launches nothing and returns None; the Python binding then
// takes the call and gives its usual errors.
//
// The workspace is grow-only per (device, stream): a buffer replaced by a
// larger one stays alive until the process ends, since a HIP graph captured
// earlier keeps its address.
//
// Reference counterpart: the pybind binding paged_decode_split of
// csrc_native/m1_binding.cpp:78-115 (checks, output and workspace, launch on
// the caller's stream).

#include <torch/extension.h>

#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <limits>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "mxfa_mi355x.h"

namespace {

struct Workspaces {
  std::mutex mu;
  std::map<std::pair<int, void *>, at::Tensor> live;
  std::vector<at::Tensor> retired;
};

// Never destroyed: the tensors must outlive every graph that holds their
// address, and static destruction at exit would run after the HIP runtime.
Workspaces &workspaces() {
  static Workspaces *w = new Workspaces();
  return *w;
}

at::Tensor workspace(const at::Device &device, void *stream, size_t bytes) {
  Workspaces &w = workspaces();
  std::lock_guard<std::mutex> lock(w.mu);
  const auto key = std::make_pair((int)device.index(), stream);
  auto it = w.live.find(key);
  if (it == w.live.end() || (size_t)it->second.numel() < bytes) {
    int64_t size = std::max<int64_t>((int64_t)bytes, 1 << 20);
    if (it != w.live.end()) {
      size = std::max<int64_t>(size, 2 * it->second.numel());
      w.retired.push_back(it->second);
    }
    at::Tensor t = at::empty({size}, at::TensorOptions().dtype(at::kByte).device(device));
    w.live[key] = t;
    return t;
  }
  return it->second;
}

// MXFA_POISON_OUTPUTS=1 (a debugging aid, read once; the Python binding reads
// the same variable): before each launch outside graph capture the output is
// filled with NaN and the workspace with 0xff bytes, so a row or a piece the
// kernels fail to write shows up as NaN rather than as a stale value.
bool poison_outputs() {
  static const bool on = [] {
    const char *e = std::getenv("MXFA_POISON_OUTPUTS");
    return e != nullptr && std::string(e) == "1";
  }();
  return on;
}

void poison(void *stream, at::Tensor &out, at::Tensor *ws) {
  // An output whose rows overlap is refused by the launch; it is not filled.
  if (!poison_outputs() || at::has_internal_overlap(out) != at::MemOverlap::No) return;
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing((hipStream_t)stream, &status) != hipSuccess ||
      status != hipStreamCaptureStatusNone)
    return;
  out.fill_(std::numeric_limits<float>::quiet_NaN());
  if (ws) ws->fill_(0xff);
}

// (bytes of the live workspaces, bytes of the retired ones)
std::pair<int64_t, int64_t> workspace_bytes() {
  Workspaces &w = workspaces();
  std::lock_guard<std::mutex> lock(w.mu);
  int64_t live = 0, retired = 0;
  for (const auto &kv : w.live) live += kv.second.numel();
  for (const auto &t : w.retired) retired += t.numel();
  return {live, retired};
}

bool aligned(const void *p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

// Compute units of a device, looked up once (the split heuristic's input).
int num_cus(int device) {
  static std::mutex mu;
  static std::map<int, int> cus;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cus.find(device);
  if (it != cus.end()) return it->second;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    n = 0;
  cus[device] = n;
  return n;
}

// q or out as [B, HQ, HD] strides (batch, head), or false when the layout is
// not [B, HQ, HD] / [B, 1, HQ, HD] with a contiguous last dim.
bool bhd_strides(const at::Tensor &t, int64_t &sb, int64_t &sh) {
  if (t.dim() == 3) {
    sb = t.stride(0);
    sh = t.stride(1);
  } else if (t.dim() == 4 && t.size(1) == 1) {
    sb = t.stride(0);
    sh = t.stride(2);
  } else {
    return false;
  }
  return t.stride(-1) == 1;
}

py::object decode(const at::Tensor &q, const at::Tensor &k_cache, const at::Tensor &v_cache,
                  const at::Tensor &block_table, const at::Tensor &cache_seqlens, double scale,
                  const c10::optional<at::Tensor> &out_arg,
                  const c10::optional<int64_t> &num_splits_arg, int64_t seqlen_add) {
  const at::ScalarType dt = q.scalar_type();
  if (dt != at::kHalf && dt != at::kBFloat16) return py::none();
  if (!q.is_cuda() || k_cache.scalar_type() != dt || v_cache.scalar_type() != dt) return py::none();
  if (k_cache.dim() != 4 || !v_cache.sizes().equals(k_cache.sizes())) return py::none();
  if (!v_cache.strides().equals(k_cache.strides()) || k_cache.stride(3) != 1) return py::none();
  if (block_table.scalar_type() != at::kInt || cache_seqlens.scalar_type() != at::kInt)
    return py::none();
  if (block_table.dim() != 2 || block_table.stride(1) != 1 || cache_seqlens.dim() != 1 ||
      !cache_seqlens.is_contiguous())
    return py::none();
  const at::Device device = q.device();
  if (k_cache.device() != device || v_cache.device() != device ||
      block_table.device() != device || cache_seqlens.device() != device)
    return py::none();
  if (device.index() != c10::hip::current_device()) return py::none();
  int64_t q_sb, q_sh;
  if (!bhd_strides(q, q_sb, q_sh)) return py::none();
  const int64_t batch = q.size(0), hq = q.size(-2), hd = q.size(-1);
  const int64_t pages = k_cache.size(0), ps = k_cache.size(1), hkv = k_cache.size(2);
  if (k_cache.size(3) != hd || block_table.size(0) != batch || cache_seqlens.size(0) != batch ||
      block_table.size(1) < 1)
    return py::none();
  // The kernels' 16-byte fragments: aligned pointers, strides of 8 elements.
  if (!aligned(q.data_ptr(), 16) || !aligned(k_cache.data_ptr(), 16) ||
      !aligned(v_cache.data_ptr(), 16) || ((q_sb | q_sh) & 7) || q_sb < 0 || q_sh < 0 ||
      (hq > 1 && q_sh < hd))
    return py::none();
  at::Tensor out;
  int64_t o_sb, o_sh;
  if (out_arg.has_value()) {
    out = *out_arg;
    if (out.scalar_type() != dt || out.device() != device || !out.sizes().equals(q.sizes()) ||
        !bhd_strides(out, o_sb, o_sh) || !aligned(out.data_ptr(), 8) || ((o_sb | o_sh) & 3))
      return py::none();
  } else {
    out = at::empty(q.sizes(), q.options());
    bhd_strides(out, o_sb, o_sh);
  }
  void *stream = (void *)c10::hip::getCurrentHIPStream(device.index()).stream();
  // No num_splits: the heuristic's choice. Values the C ABI rejects (0, below
  // MXFA_SPLITS_PER_SEQUENCE, above 65535) go to the binding's path, which
  // reports them.
  int ns = 0;
  if (num_splits_arg.has_value()) {
    const int64_t v = *num_splits_arg;
    if ((v <= 0 && v != MXFA_SPLITS_PER_SEQUENCE) || v > 65535) return py::none();
    ns = (int)v;
  } else if (mxfa_split_heuristic((int)batch, (int)hq, (int)hkv, (int)hd, (int)ps,
                                  (int)block_table.size(1), num_cus(device.index()),
                                  &ns) != MXFA_OK) {
    return py::none();
  }
  size_t ws_bytes = 0;
  if (mxfa_split_decode_workspace_size((int)batch, (int)hq, (int)hd, ns, &ws_bytes) != MXFA_OK)
    return py::none();
  at::Tensor ws_t;
  if (ws_bytes) ws_t = workspace(device, stream, ws_bytes);
  void *ws = ws_bytes ? ws_t.data_ptr() : nullptr;
  poison(stream, out, ws_bytes ? &ws_t : nullptr);
  const int rc = mxfa_split_decode_launch(
      q.data_ptr(), q_sb, q_sh, k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
      k_cache.stride(1), k_cache.stride(2), block_table.data_ptr<int32_t>(), block_table.stride(0),
      cache_seqlens.data_ptr<int32_t>(), (int)seqlen_add, out.data_ptr(), o_sb, o_sh, ws, ws_bytes,
      (float)scale, (int)batch, (int)hq, (int)hkv, (int)hd, (int)ps, (int)block_table.size(1),
      (int)pages, dt == at::kBFloat16 ? MXFA_DTYPE_BF16 : MXFA_DTYPE_F16, ns, stream);
  if (rc == MXFA_EUNSUPPORTED || rc == MXFA_EINVAL) return py::none();  // nothing launched
  if (rc != MXFA_OK)
    throw std::runtime_error(std::string("mxfa_split_decode_launch failed (") +
                             std::to_string(rc) + "): " + mxfa_strerror(rc));
  return py::cast(out);
}

// reshape_and_cache(key, value, key_cache, value_cache, slot_mapping): the
// vLLM-form append of 16-bit caches (mxfa_reshape_and_cache_launch) for the
// common call: key/value [T, HKV, HD] sharing strides with a contiguous last
// dim, caches [pages, PS, HKV, HD] of their dtype sharing strides, int64
// contiguous slots (at least T of them), every tensor on the current GPU.
// Returns true once launched on torch's current stream; false (nothing
// launched) for any other call, which the Python binding then takes.
bool reshape_and_cache(const at::Tensor &key, const at::Tensor &value,
                       const at::Tensor &key_cache, const at::Tensor &value_cache,
                       const at::Tensor &slot_mapping) {
  const at::ScalarType dt = key.scalar_type();
  if (dt != at::kHalf && dt != at::kBFloat16) return false;
  if (!key.is_cuda() || value.scalar_type() != dt || key_cache.scalar_type() != dt ||
      value_cache.scalar_type() != dt || slot_mapping.scalar_type() != at::kLong)
    return false;
  if (key.dim() != 3 || !value.sizes().equals(key.sizes()) || !value.strides().equals(key.strides()) ||
      key.stride(2) != 1)
    return false;
  if (key_cache.dim() != 4 || !value_cache.sizes().equals(key_cache.sizes()) ||
      !value_cache.strides().equals(key_cache.strides()) || key_cache.stride(3) != 1)
    return false;
  if (key.size(1) != key_cache.size(2) || key.size(2) != key_cache.size(3)) return false;
  if (slot_mapping.dim() != 1 || !slot_mapping.is_contiguous() ||
      slot_mapping.size(0) < key.size(0))
    return false;
  const at::Device device = key.device();
  if (value.device() != device || key_cache.device() != device ||
      value_cache.device() != device || slot_mapping.device() != device ||
      device.index() != c10::hip::current_device())
    return false;
  void *stream = (void *)c10::hip::getCurrentHIPStream(device.index()).stream();
  const int rc = mxfa_reshape_and_cache_launch(
      key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1), key_cache.data_ptr(),
      value_cache.data_ptr(), key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
      slot_mapping.data_ptr<int64_t>(), (int)key.size(0), (int)key.size(1), (int)key.size(2),
      (int)key_cache.size(1), (int)key_cache.size(0),
      dt == at::kBFloat16 ? MXFA_DTYPE_BF16 : MXFA_DTYPE_F16, stream);
  if (rc == MXFA_EUNSUPPORTED || rc == MXFA_EINVAL) return false;  // nothing launched
  if (rc != MXFA_OK)
    throw std::runtime_error(std::string("mxfa_reshape_and_cache_launch failed (") +
                             std::to_string(rc) + "): " + mxfa_strerror(rc));
  return true;
}

}  // namespace

PYBIND11_MODULE(_mxfa_torch, m) {
  m.doc() = "torch operator in front of libmxfa_mi355x's split decode C ABI";
  m.def("decode", &decode, py::arg("q"), py::arg("k_cache"), py::arg("v_cache"),
        py::arg("block_table"), py::arg("cache_seqlens"), py::arg("scale"),
        py::arg("out") = py::none(), py::arg("num_splits") = py::none(),
        py::arg("seqlen_add") = 0);
  m.def("reshape_and_cache", &reshape_and_cache, py::arg("key"), py::arg("value"),
        py::arg("key_cache"), py::arg("value_cache"), py::arg("slot_mapping"));
  m.def("abi_version", &mxfa_abi_version);
  m.def("workspace_bytes", &workspace_bytes,
        "(bytes of live workspaces, bytes of workspaces replaced by larger ones)");
}
