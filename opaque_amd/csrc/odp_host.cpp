// Host-side bookkeeping for GhostPlan.rebind: reading the structure and the
// addresses of a call's LoRA site tensors, and making the output leaf views.
// No device work; torch is used only to read tensor metadata and make views.
//
// A plan built for one call is re-pointed at the next call's inputs when
// their structure is the same (shapes, strides, dtypes, devices, 16-byte
// alignment, which sites share an activation, the sites' scalars).  Doing
// that per seam in Python costs a few microseconds per tensor, which for a
// 224-seam model is a tenth of the DP step; here it is a few nanoseconds.
#include <torch/csrc/autograd/python_variable.h>
#include <torch/extension.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace py = pybind11;

namespace {

constexpr int kMaxDims = 6;

void put(std::string& out, int64_t v) { out.append(reinterpret_cast<const char*>(&v), sizeof v); }

// Shape, strides, dtype, device and address alignment of a tensor.
void put_tensor(std::string& out, const at::Tensor& t) {
  const int64_t nd = t.dim();
  TORCH_CHECK(nd <= kMaxDims, "site tensors have at most ", kMaxDims, " dimensions");
  put(out, nd);
  for (int64_t i = 0; i < nd; ++i) put(out, t.size(i));
  for (int64_t i = 0; i < nd; ++i) put(out, t.stride(i));
  put(out, static_cast<int64_t>(t.scalar_type()));
  put(out, t.is_cuda() ? static_cast<int64_t>(t.get_device()) : -1);
  put(out, reinterpret_cast<int64_t>(t.data_ptr()) & 15);
}

// Shape and device only (B is copied into a buffer of the activation's dtype
// unless it can be read in place, which its dtype and contiguity decide).
void put_shape_device(std::string& out, const at::Tensor& t) {
  put(out, t.dim());
  for (int64_t i = 0; i < t.dim(); ++i) put(out, t.size(i));
  put(out, t.is_cuda() ? static_cast<int64_t>(t.get_device()) : -1);
}

// Attribute names, made once (a lookup by a C string builds a new str each time).
struct Names {
  py::str segments{"segments"}, x{"x"}, g{"g"}, A{"A"}, B{"B"}, scaling{"scaling"}, a_leaf{"a_leaf"},
      b_leaf{"b_leaf"}, a_transposed{"a_transposed"}, b_transposed{"b_transposed"}, v{"v"}, u{"u"};
};
const Names& names() {
  static const Names* n = new Names();  // never destroyed: outlives the interpreter's teardown order
  return *n;
}

// An attribute of a site object from its instance dict (the sites are plain
// dataclass instances; the dict lookup skips the type's attribute search).
PyObject* field(PyObject* d, const py::str& name) {
  PyObject* v = PyDict_GetItemWithError(d, name.ptr());
  if (v == nullptr) {
    if (PyErr_Occurred()) throw py::error_already_set();
    throw py::key_error(std::string("site has no attribute ") + std::string(py::str(name)));
  }
  return v;
}

const at::Tensor& tensor_field(PyObject* d, const py::str& name) {
  PyObject* v = field(d, name);
  TORCH_CHECK(THPVariable_Check(v), "site attribute ", std::string(py::str(name)), " is not a tensor");
  return THPVariable_Unpack(v);
}

int64_t leaf_field(PyObject* d, const py::str& name) {
  PyObject* v = field(d, name);
  return v == Py_None ? -1 : PyLong_AsLongLong(v);
}

// An optional tensor attribute (the seam's rank-space products): its key, or
// a marker when absent; returns its address or 0.
int64_t put_optional(std::string& out, PyObject* d, const py::str& name) {
  PyObject* v = field(d, name);
  if (v == Py_None) {
    put(out, -1);
    return 0;
  }
  TORCH_CHECK(THPVariable_Check(v), "site attribute ", std::string(py::str(name)), " is not a tensor");
  const at::Tensor& t = THPVariable_Unpack(v);
  put_tensor(out, t);
  return reinterpret_cast<int64_t>(t.data_ptr());
}

constexpr int64_t kPtrs = 6;  // x, g, A, B, v, u per site

// Structure of a list of LoraSite objects as bytes, and per site the
// addresses of x, g, A, B, v and u (0 when absent) written to `ptrs` (an
// int64 CPU tensor of 6 x the number of sites).  Returns None when a site
// brings its own segments (the caller then takes the general path).
py::object lora_signature(py::list sites, at::Tensor ptrs) {
  const int64_t n = static_cast<int64_t>(sites.size());
  TORCH_CHECK(ptrs.scalar_type() == at::kLong && ptrs.is_contiguous() && !ptrs.is_cuda() &&
                  ptrs.numel() >= kPtrs * n,
              "ptrs must be a contiguous int64 CPU tensor of at least 6 entries per site");
  int64_t* P = ptrs.data_ptr<int64_t>();
  std::string sig;
  sig.reserve(static_cast<size_t>(n) * 400);
  std::unordered_map<int64_t, int64_t> first;  // activation address -> index of its first distinct key
  std::vector<std::string> xkeys;
  const Names& nm = names();
  const c10::TensorImpl* last_x = nullptr;
  int64_t last_idx = 0;
  for (int64_t i = 0; i < n; ++i) {
    PyObject* s = PyList_GET_ITEM(sites.ptr(), i);
    PyObject** dp = _PyObject_GetDictPtr(s);
    TORCH_CHECK(dp != nullptr && *dp != nullptr, "sites must be LoraSite instances");
    PyObject* d = *dp;
    if (field(d, nm.segments) != Py_None) return py::none();
    const at::Tensor& x = tensor_field(d, nm.x);
    const at::Tensor& g = tensor_field(d, nm.g);
    const at::Tensor& A = tensor_field(d, nm.A);
    const at::Tensor& B = tensor_field(d, nm.B);
    const int64_t xp = reinterpret_cast<int64_t>(x.data_ptr());
    if (x.unsafeGetTensorImpl() == last_x) {
      put(sig, last_idx);  // the previous site's tensor object: same key, same index
    } else {
      std::string xk;
      put_tensor(xk, x);
      auto it = first.find(xp);
      if (it == first.end()) {
        last_idx = static_cast<int64_t>(xkeys.size());
        first.emplace(xp, last_idx);
        xkeys.push_back(std::move(xk));
        put(sig, last_idx);
        last_x = x.unsafeGetTensorImpl();
      } else if (xkeys[it->second] == xk) {
        last_idx = it->second;
        put(sig, last_idx);
        last_x = x.unsafeGetTensorImpl();
      } else {  // another view at the same address
        put(sig, -1 - it->second);
        sig += xk;
        last_x = nullptr;
      }
    }
    put_tensor(sig, g);
    put_tensor(sig, A);  // read in place with the strides and dtype of the pack table
    put_shape_device(sig, B);
    put(sig, static_cast<int64_t>(B.scalar_type()));
    put(sig, B.is_contiguous() ? 1 : 0);
    double scaling = PyFloat_AsDouble(field(d, nm.scaling));
    if (scaling == -1.0 && PyErr_Occurred()) throw py::error_already_set();
    int64_t sbits;
    std::memcpy(&sbits, &scaling, sizeof sbits);
    put(sig, sbits);
    put(sig, leaf_field(d, nm.a_leaf));
    put(sig, leaf_field(d, nm.b_leaf));
    put(sig, (PyObject_IsTrue(field(d, nm.a_transposed)) ? 1 : 0) | (PyObject_IsTrue(field(d, nm.b_transposed)) ? 2 : 0));
    int64_t* Pi = P + kPtrs * i;
    Pi[0] = xp;
    Pi[1] = reinterpret_cast<int64_t>(g.data_ptr());
    Pi[2] = reinterpret_cast<int64_t>(A.data_ptr());
    Pi[3] = reinterpret_cast<int64_t>(B.data_ptr());
    Pi[4] = put_optional(sig, d, nm.v);
    Pi[5] = put_optional(sig, d, nm.u);
  }
  // The distinct activations' keys close the signature.
  put(sig, static_cast<int64_t>(xkeys.size()));
  for (const auto& k : xkeys) sig += k;
  return py::bytes(sig);
}

// Views of flat output buffers: leaf i is buffers[buf[i]] seen with
// sizes[i] / strides[i] at element offset off[i], in the dtype of
// dtypes[i] (a tensor of that dtype; by default the buffer's own, and
// offsets then count the buffer's elements).  Built once per plan.
class ViewMaker {
 public:
  ViewMaker(std::vector<int64_t> buf, std::vector<std::vector<int64_t>> sizes,
            std::vector<std::vector<int64_t>> strides, std::vector<int64_t> off,
            std::vector<at::Tensor> dtypes = {})
      : buf_(std::move(buf)), sizes_(std::move(sizes)), strides_(std::move(strides)), off_(std::move(off)) {
    TORCH_CHECK(buf_.size() == sizes_.size() && buf_.size() == strides_.size() && buf_.size() == off_.size(),
                "ViewMaker: one buffer index, shape, stride list and offset per leaf");
    TORCH_CHECK(dtypes.empty() || dtypes.size() == buf_.size(), "ViewMaker: one dtype per leaf, or none");
    for (const auto& t : dtypes) dtypes_.push_back(t.dtype());
  }
  // Each leaf is a tensor over its buffer's storage, made directly (no
  // operator dispatch, no autograd view record: the leaves are outputs).
  std::vector<at::Tensor> make(const std::vector<at::Tensor>& buffers) const {
    for (const auto& b : buffers) TORCH_CHECK(!b.requires_grad(), "ViewMaker: buffers must not require grad");
    std::vector<at::Tensor> out;
    out.reserve(buf_.size());
    for (size_t i = 0; i < buf_.size(); ++i) {
      const at::Tensor& b = buffers.at(static_cast<size_t>(buf_[i]));
      TORCH_CHECK(b.is_contiguous() && b.dim() == 1, "ViewMaker: flat contiguous buffers only");
      const caffe2::TypeMeta dt = dtypes_.empty() ? b.dtype() : dtypes_[i];
      const int64_t base_bytes = b.storage_offset() * static_cast<int64_t>(b.dtype().itemsize());
      TORCH_CHECK(base_bytes % static_cast<int64_t>(dt.itemsize()) == 0, "ViewMaker: misaligned dtype view");
      at::Tensor t = at::detail::make_tensor<c10::TensorImpl>(c10::Storage(b.storage()), b.key_set(), dt);
      t.unsafeGetTensorImpl()->set_sizes_and_strides(sizes_[i], strides_[i],
                                                     base_bytes / static_cast<int64_t>(dt.itemsize()) + off_[i]);
      out.push_back(std::move(t));
    }
    return out;
  }

 private:
  std::vector<int64_t> buf_;
  std::vector<std::vector<int64_t>> sizes_, strides_;
  std::vector<int64_t> off_;
  std::vector<caffe2::TypeMeta> dtypes_;
};

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Host-side helpers of opaque_amd's plan reuse (no device work).";
  m.def("lora_signature", &lora_signature, py::arg("sites"), py::arg("ptrs"));
  py::class_<ViewMaker>(m, "ViewMaker")
      .def(py::init<std::vector<int64_t>, std::vector<std::vector<int64_t>>, std::vector<std::vector<int64_t>>,
                    std::vector<int64_t>, std::vector<at::Tensor>>(),
           py::arg("buf"), py::arg("sizes"), py::arg("strides"), py::arg("off"),
           py::arg("dtypes") = std::vector<at::Tensor>{})
      .def("make", &ViewMaker::make);
}
