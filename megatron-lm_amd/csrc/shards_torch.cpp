// Python binding of the flat-shard entry points (ec_xor_encode, ec_rs_encode,
// ec_rs_decode) that takes torch tensors directly, and the address and size
// reads of the ragged tensor lists.
//
// codec.matvec / codec.xor_encode call it once per call: the checks on every
// shard (device tensor, contiguous, one device, one byte size), the host
// arrays of device addresses, the output allocation and the lookup of torch's
// current stream all happen here, in one crossing from Python.  Done in
// Python through ctypes they cost about 10 us per call, more than the kernel
// over a few MiB shards.
//
// The C ABI (include/ec_mi355.h) stays free of torch types; this module is a
// client of it, like the ctypes binding, and links libec_mi355.so.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "ec_mi355.h"

namespace {

enum Op : int64_t { kXor = 0, kEncode = 1, kDecode = 2 };

// Byte size of a tensor that the kernels may read or write through its data
// pointer; throws ValueError (the Python checks' wording) otherwise.
int64_t checked_bytes(const at::Tensor& t, const char* what, size_t i,
                      const c10::Device& device) {
  if (!t.is_cuda())
    throw py::value_error(std::string(what) + "[" + std::to_string(i) +
                          "] must be a device (HIP) tensor");
  if (!t.is_contiguous())
    throw py::value_error(std::string(what) + "[" + std::to_string(i) + "] must be contiguous");
  if (t.device() != device)
    throw py::value_error(std::string(what) + "[" + std::to_string(i) + "] is on " +
                          t.device().str() + ", the other operands on " + device.str());
  return static_cast<int64_t>(t.nbytes());
}

// out[i] = XOR_j coeff[i*k + j] * shards[j] (op kEncode / kDecode, coeff the
// m x k bytes), or out[0] = XOR_j shards[j] (op kXor, coeff ignored).  `out`
// None allocates the outputs; `stream` None is torch's current stream of the
// shards' device.  Returns (status, outputs): the status of the C call, for
// the caller to turn into its error type.
py::tuple shard_call(int64_t op, const std::string& coeff, int64_t m,
                     const std::vector<at::Tensor>& shards,
                     std::optional<std::vector<at::Tensor>> out,
                     std::optional<int64_t> stream) {
  if (op != kXor && op != kEncode && op != kDecode)
    throw py::value_error("unknown shard operation " + std::to_string(op));
  const size_t k = shards.size();
  if (k == 0) throw py::value_error("no shards");
  if (op == kXor) {
    m = 1;
  } else if (m <= 0 || coeff.size() != static_cast<size_t>(m) * k) {
    throw py::value_error("coefficient matrix has " +
                          std::to_string(m > 0 ? coeff.size() / static_cast<size_t>(m) : 0) +
                          " columns, got " + std::to_string(k) + " shards");
  }
  const c10::Device device = shards[0].device();
  std::vector<const uint8_t*> in_ptrs(k);
  int64_t nbytes = -1;
  for (size_t j = 0; j < k; ++j) {
    const int64_t nb = checked_bytes(shards[j], "shards", j, device);
    if (nbytes < 0) nbytes = nb;
    if (nb != nbytes)
      throw py::value_error("shards differ in byte size: " + std::to_string(nbytes) + " and " +
                            std::to_string(nb));
    in_ptrs[j] = static_cast<const uint8_t*>(shards[j].data_ptr());
  }
  std::vector<at::Tensor> outs;
  if (out.has_value()) {
    outs = *out;
    if (outs.size() != static_cast<size_t>(m))
      throw py::value_error("out: expected " + std::to_string(m) + " tensors, got " +
                            std::to_string(outs.size()));
    for (size_t i = 0; i < outs.size(); ++i) {
      const int64_t nb = checked_bytes(outs[i], "out", i, device);
      if (nb != nbytes)
        throw py::value_error("out[" + std::to_string(i) + "] has " + std::to_string(nb) +
                              " bytes, shards have " + std::to_string(nbytes));
    }
  } else {
    const auto opts = at::TensorOptions().dtype(at::kByte).device(device);
    outs.reserve(static_cast<size_t>(m));
    for (int64_t i = 0; i < m; ++i) outs.push_back(at::empty({nbytes}, opts));
  }
  std::vector<uint8_t*> out_ptrs(outs.size());
  for (size_t i = 0; i < outs.size(); ++i) out_ptrs[i] = static_cast<uint8_t*>(outs[i].data_ptr());
  ec_stream_t s = stream.has_value()
                      ? reinterpret_cast<ec_stream_t>(static_cast<intptr_t>(*stream))
                      : reinterpret_cast<ec_stream_t>(
                            c10::hip::getCurrentHIPStream(device.index()).stream());
  const uint64_t n = static_cast<uint64_t>(nbytes);
  const auto* cf = reinterpret_cast<const uint8_t*>(coeff.data());
  int status;
  {
    py::gil_scoped_release nogil;
    if (op == kXor)
      status = ec_xor_encode(in_ptrs.data(), static_cast<int>(k), out_ptrs[0], n, s);
    else if (op == kEncode)
      status = ec_rs_encode(cf, static_cast<int>(k), static_cast<int>(m), in_ptrs.data(),
                            out_ptrs.data(), n, s);
    else
      status = ec_rs_decode(cf, static_cast<int>(k), static_cast<int>(m), in_ptrs.data(),
                            out_ptrs.data(), n, s);
  }
  return py::make_tuple(status, outs);
}

// (base addresses, byte sizes) of a list of tensors that must all be
// contiguous device tensors on device `device`, as two byte strings of
// uint64 / int64 (numpy reads them without a copy).  The ragged-list
// layout checks every tensor of a checkpoint (thousands) on the path that
// holds training: here that costs the list conversion, about 0.1 us per
// tensor, against 0.36 us in Python.
py::tuple spans(const std::vector<at::Tensor>& tensors, int64_t device) {
  const size_t n = tensors.size();
  std::string base(n * sizeof(uint64_t), '\0'), size(n * sizeof(int64_t), '\0');
  auto* b = reinterpret_cast<uint64_t*>(&base[0]);
  auto* z = reinterpret_cast<int64_t*>(&size[0]);
  for (size_t i = 0; i < n; ++i) {
    const at::Tensor& t = tensors[i];
    if (!t.is_cuda())
      throw py::value_error("tensors[" + std::to_string(i) + "] must be a device (HIP) tensor");
    if (!t.is_contiguous())
      throw py::value_error("tensors[" + std::to_string(i) + "] must be contiguous");
    if (t.device().index() != device)
      throw py::value_error("tensors[" + std::to_string(i) + "] is on " + t.device().str() +
                            ", the other operands on cuda:" + std::to_string(device));
    b[i] = static_cast<uint64_t>(reinterpret_cast<uintptr_t>(t.data_ptr()));
    z[i] = static_cast<int64_t>(t.nbytes());
  }
  return py::make_tuple(py::bytes(base), py::bytes(size));
}

// The raw handle of torch's current stream on a device (-1: the current
// device), as codec.stream_handle passes it to the C ABI.
int64_t current_stream(int64_t device) {
  return static_cast<int64_t>(reinterpret_cast<intptr_t>(
      c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream()));
}

}  // namespace

PYBIND11_MODULE(_ec_shards, mod) {
  mod.doc() = "torch-tensor binding of the flat-shard calls of libec_mi355.so";
  mod.attr("XOR") = static_cast<int64_t>(kXor);
  mod.attr("ENCODE") = static_cast<int64_t>(kEncode);
  mod.attr("DECODE") = static_cast<int64_t>(kDecode);
  mod.def("shard_call", &shard_call, py::arg("op"), py::arg("coeff"), py::arg("m"),
          py::arg("shards"), py::arg("out") = py::none(), py::arg("stream") = py::none());
  mod.def("current_stream", &current_stream, py::arg("device") = -1);
  mod.def("spans", &spans, py::arg("tensors"), py::arg("device"));
}
