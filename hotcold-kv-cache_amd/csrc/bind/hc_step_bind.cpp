// Native per-step half of the packed append+decode call
// (hc_decode_attn_append_packed, include/hotcold_hip.h), for the Python
// decode loop: one call per layer and token.
//
// The caller (hotcold_kv/ops.py, _AppendPlan) keeps one hc_decode_append_args
// struct per hot-buffer storage with everything that does not change from
// step to step (shape, base pointers, strides, dtype, workspace, held slot,
// scaling).  This function takes the step's tensors, checks them against the
// struct's shape, dtype and device, writes their pointers and strides into
// the struct, allocates the output and launches.  It does in C++ what the
// Python plan did per call (three to five row checks, the output's
// allocation, the ctypes call); the launch itself is the library's.
//
// Host code only: it is built against torch's headers as a Python extension
// module and calls the already-loaded libhotcold_hip.so, whose symbols the
// Python side loads with RTLD_GLOBAL.  No torch type crosses the C ABI.
#include <torch/extension.h>

#include <string>

#include "hotcold_hip.h"

namespace {

at::ScalarType scalar_type(int64_t code) {
  switch (code) {
    case HC_DTYPE_F32: return at::kFloat;
    case HC_DTYPE_F16: return at::kHalf;
    case HC_DTYPE_BF16: return at::kBFloat16;
    default: TORCH_CHECK(false, "decode_append_rows: unknown dtype code ", code);
  }
  return at::kFloat;
}

// A (B, H, D) or (B, H, 1, D) row tensor of the step: pointer and (batch,
// head) strides, after the checks the Python plan made (same messages).
void row(const at::Tensor& t, int64_t B, int64_t H, int64_t D, at::ScalarType st, int64_t dev, const char* what,
         const void** ptr, int64_t* sb, int64_t* sh) {
  const auto sizes = t.sizes();
  const bool shape_ok = (sizes.size() == 3 && sizes[0] == B && sizes[1] == H && sizes[2] == D) ||
                        (sizes.size() == 4 && sizes[0] == B && sizes[1] == H && sizes[2] == 1 && sizes[3] == D);
  const bool ok = shape_ok && t.scalar_type() == st && t.is_cuda() && t.get_device() == dev;
  TORCH_CHECK(ok, "decode_append_rows: ", what, " must be (", B, ", ", H, ", ", D, ") or (", B, ", ", H, ", 1, ", D,
              ") device rows in the buffer's dtype ", c10::toString(st), "; got ", t.sizes(), " ",
              c10::toString(t.scalar_type()), " on ", t.device());
  const auto strides = t.strides();
  TORCH_CHECK(strides.back() == 1, "decode_append_rows: ", what, " needs a unit last stride");
  *ptr = t.data_ptr();
  *sb = strides[0];
  *sh = strides[1];
}

}  // namespace

// Returns (out, status): status is the library's (0, or HC_ERR_WORKSPACE for
// a workspace the caller must grow before calling again, or another error
// whose text hc_last_error() holds).  p_new / pos_new given means the
// struct's p_dst / pos_dst already point at row S-1's destination.
std::tuple<at::Tensor, int64_t> decode_append_step(int64_t args_addr, const at::Tensor& q, const at::Tensor& k_new,
                                                   const at::Tensor& v_new, const c10::optional<at::Tensor>& p_new,
                                                   const c10::optional<at::Tensor>& pos_new, bool keepdim,
                                                   int64_t stream, int64_t device_index) {
  auto* a = reinterpret_cast<hc_decode_append_args*>(args_addr);
  const at::ScalarType st = scalar_type(a->dtype);
  row(q, a->B, a->Hq, a->D, st, device_index, "q", &a->q, &a->q_sb, &a->q_sh);
  row(k_new, a->B, a->Hk, a->D, st, device_index, "k_new", &a->k_new, &a->kn_sb, &a->kn_sh);
  row(v_new, a->B, a->Hk, a->D, st, device_index, "v_new", &a->v_new, &a->vn_sb, &a->vn_sh);
  if (p_new.has_value()) {
    row(*p_new, a->B, a->Hk, a->D, st, device_index, "p_new", &a->p_new, &a->pn_sb, &a->pn_sh);
  } else {
    a->p_new = nullptr;
    a->p_dst = nullptr;
  }
  if (pos_new.has_value()) {
    const at::Tensor& p = *pos_new;
    TORCH_CHECK(p.scalar_type() == at::kLong && p.dim() >= 1 && p.size(0) == a->B && p.is_cuda() &&
                    p.get_device() == device_index,
                "decode_append_rows: pos_new must be (B,1) int64");
    a->pos_new = p.data_ptr<int64_t>();
    a->posn_sb = p.stride(0);
  } else {
    a->pos_new = nullptr;
    a->pos_dst = nullptr;
  }
  at::Tensor out = keepdim ? at::empty({a->B, a->Hq, 1, a->D}, q.options()) : at::empty({a->B, a->Hq, a->D}, q.options());
  a->out = out.data_ptr();
  const int rc = hc_decode_attn_append_packed(a, reinterpret_cast<void*>(stream));
  return {out, (int64_t)rc};
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("decode_append_step", &decode_append_step, "the per-step half of hc_decode_attn_append_packed");
}
