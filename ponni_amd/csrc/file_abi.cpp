// C ABI over the header-only .ponni reader/writer (ponni_amd/include/ponni/ponni_file.h).
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ponni_hip.h"
#include "../include/ponni/ponni_file.h"

namespace ponni_hip {
int set_error(int status, std::string const& message);
}

extern "C" {

uint64_t ponni_fnv1a64(const void* data, size_t size) {
  return ponni::ponni_fnv1a64(static_cast<unsigned char const*>(data), size);
}

// "ponni-template-model-v1\n" + "I\tlabel\tnin\tnout\tntrainable\n" per layer
// (ponni_Inference.h:270-288).
int ponni_template_fingerprint(int32_t num_layers, const char* const* labels, const int32_t* num_inputs,
                               const int32_t* num_outputs, const int64_t* num_trainable, char* out, size_t out_len) {
  if (num_layers <= 0 || !labels || !num_inputs || !num_outputs || !num_trainable || !out)
    return ponni_hip::set_error(PONNI_ERR_INVALID_ARGUMENT, "invalid fingerprint arguments");
  std::string text = "ponni-template-model-v1\n";
  for (int32_t i = 0; i < num_layers; i++) {
    text += std::to_string(i) + '\t' + (labels[i] ? labels[i] : "") + '\t' + std::to_string(num_inputs[i]) + '\t' +
            std::to_string(num_outputs[i]) + '\t' + std::to_string(num_trainable[i]) + '\n';
  }
  std::string const fp = ponni::ponni_fnv1a64_string(
      ponni::ponni_fnv1a64(reinterpret_cast<unsigned char const*>(text.data()), text.size()));
  if (out_len < fp.size() + 1) return ponni_hip::set_error(PONNI_ERR_INVALID_ARGUMENT, "fingerprint buffer too small");
  std::memcpy(out, fp.c_str(), fp.size() + 1);
  return PONNI_OK;
}

int ponni_file_write_parameters(const char* path, const char* model_fingerprint, const void* values, int64_t count,
                                int32_t elem_size, const char* target) {
  if (!path || !model_fingerprint || (!values && count > 0) || count <= 0 || (elem_size != 4 && elem_size != 8))
    return ponni_hip::set_error(PONNI_ERR_INVALID_ARGUMENT, "invalid .ponni write arguments");
  std::string error;
  std::vector<ponni::PonniTensorSpec> specs{
      {"parameters", elem_size == 8 ? "F64" : "F32", {static_cast<std::size_t>(count)}, 0}};
  bool const ok = elem_size == 8
                      ? ponni::write_ponni_file(path, specs, model_fingerprint, static_cast<double const*>(values),
                                                &error, target ? target : "ponni")
                      : ponni::write_ponni_file(path, specs, model_fingerprint, static_cast<float const*>(values),
                                                &error, target ? target : "ponni");
  return ok ? PONNI_OK : ponni_hip::set_error(PONNI_ERR_IO, error);
}

int ponni_file_read_parameters(const char* path, const char* model_fingerprint, void* values, int64_t count,
                               int32_t elem_size) {
  if (!path || !model_fingerprint || !values || count <= 0 || (elem_size != 4 && elem_size != 8))
    return ponni_hip::set_error(PONNI_ERR_INVALID_ARGUMENT, "invalid .ponni read arguments");
  ponni::PonniFile file;
  std::string error;
  if (!file.load(path, &error)) return ponni_hip::set_error(PONNI_ERR_IO, error);
  std::vector<ponni::PonniTensorSpec> const expected{
      {"parameters", elem_size == 8 ? "F64" : "F32", {static_cast<std::size_t>(count)}, 0}};
  if (!file.validate(expected, model_fingerprint, &error)) return ponni_hip::set_error(PONNI_ERR_IO, error);
  auto const* t = file.find("parameters");
  unsigned char const* bytes = file.tensor_data(*t);
  if (elem_size == 8) {
    auto* v = static_cast<double*>(values);
    for (int64_t i = 0; i < count; i++) v[i] = ponni::detail::read_le<double>(bytes + 8 * i);
  } else {
    auto* v = static_cast<float*>(values);
    for (int64_t i = 0; i < count; i++) v[i] = ponni::detail::read_le<float>(bytes + 4 * i);
  }
  return PONNI_OK;
}

namespace {

bool to_specs(const ponni_tensor_spec* specs, int32_t n, int32_t elem_size, std::vector<ponni::PonniTensorSpec>& out,
              std::string& error) {
  out.clear();
  for (int32_t i = 0; i < n; i++) {
    ponni_tensor_spec const& s = specs[i];
    if (!s.name || s.rank < 0 || s.rank > 8 || s.offset < 0) {
      error = "invalid tensor spec " + std::to_string(i);
      return false;
    }
    ponni::PonniTensorSpec t{s.name, elem_size == 8 ? "F64" : "F32", {}, static_cast<std::size_t>(s.offset)};
    for (int32_t d = 0; d < s.rank; d++) {
      if (s.shape[d] < 0) {
        error = "negative dimension in tensor spec " + std::string(s.name);
        return false;
      }
      t.shape.push_back(static_cast<std::size_t>(s.shape[d]));
    }
    out.push_back(std::move(t));
  }
  return true;
}

std::size_t elements(ponni::PonniTensorSpec const& s) {
  std::size_t n = 1;
  for (std::size_t d : s.shape) n *= d;
  return n;
}

}  // namespace

int ponni_file_write_tensors(const char* path, const char* model_fingerprint, const ponni_tensor_spec* specs,
                             int32_t num_specs, const double* storage, int32_t stored_elem_size,
                             const char* source_framework, const char* target) {
  if (!path || !model_fingerprint || !specs || num_specs <= 0 || !storage ||
      (stored_elem_size != 4 && stored_elem_size != 8))
    return ponni_hip::set_error(PONNI_ERR_INVALID_ARGUMENT, "invalid .ponni write arguments");
  std::vector<ponni::PonniTensorSpec> list;
  std::string error;
  if (!to_specs(specs, num_specs, stored_elem_size, list, error))
    return ponni_hip::set_error(PONNI_ERR_INVALID_ARGUMENT, error);
  std::size_t total = 0;
  for (auto const& t : list) total = std::max(total, t.source_element_offset + elements(t));
  bool ok;
  std::string const tgt = target ? target : "generated";
  std::string const src = source_framework ? source_framework : "ponni-cpp";
  if (stored_elem_size == 8) {
    ok = ponni::write_ponni_file(path, list, model_fingerprint, storage, &error, tgt, src);
  } else {
    std::vector<float> f(storage, storage + total);
    ok = ponni::write_ponni_file(path, list, model_fingerprint, f.data(), &error, tgt, src);
  }
  return ok ? PONNI_OK : ponni_hip::set_error(PONNI_ERR_IO, error);
}

int ponni_file_read_tensors(const char* path, const char* model_fingerprint, const ponni_tensor_spec* specs,
                            int32_t num_specs, double* storage, int32_t stored_elem_size) {
  if (!path || !model_fingerprint || !specs || num_specs <= 0 || !storage ||
      (stored_elem_size != 4 && stored_elem_size != 8))
    return ponni_hip::set_error(PONNI_ERR_INVALID_ARGUMENT, "invalid .ponni read arguments");
  std::vector<ponni::PonniTensorSpec> list;
  std::string error;
  if (!to_specs(specs, num_specs, stored_elem_size, list, error))
    return ponni_hip::set_error(PONNI_ERR_INVALID_ARGUMENT, error);
  ponni::PonniFile file;
  if (!file.load(path, &error)) return ponni_hip::set_error(PONNI_ERR_IO, error);
  if (!file.validate(list, model_fingerprint, &error)) return ponni_hip::set_error(PONNI_ERR_IO, error);
  for (auto const& spec : list) {
    unsigned char const* bytes = file.tensor_data(*file.find(spec.name));
    std::size_t const n = elements(spec);
    double* dst = storage + spec.source_element_offset;
    for (std::size_t i = 0; i < n; i++)
      dst[i] = stored_elem_size == 8 ? ponni::detail::read_le<double>(bytes + 8 * i)
                                     : static_cast<double>(ponni::detail::read_le<float>(bytes + 4 * i));
  }
  return PONNI_OK;
}

}  // extern "C"
