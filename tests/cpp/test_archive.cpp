// C++17 archive boundary test: drives include/infer/archive_hip.hpp the way
// the reference's gtest suite drives infer::ModelArchive
// (tests/test_core.cpp:23-118) and the exporter's self-tests
// (tools/export_model.py:414-522).  Host-only: needs no GPU.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "infer/archive_hip.hpp"

namespace {

int failures = 0;

void expect(bool ok, const char* what) {
  if (!ok) {
    std::printf("FAILED: %s\n", what);
    ++failures;
  }
}

#pragma pack(push, 1)
struct Header {
  char magic[8];
  uint32_t version;
  uint32_t json_size;
  uint64_t data_offset;
  uint64_t reserved;
};
#pragma pack(pop)

// tests/test_core.cpp:23-63: data offset 512, one BF16 record "weight" [2].
void write_bf16_fixture(const std::string& path, const char* magic = "QWENBIN1") {
  const std::string meta =
      "{\"format\":\"QWENBIN1\",\"precision\":\"w16a16\",\"tensors\":[{\"dtype\":\"bfloat16\","
      "\"name\":\"weight\",\"nbytes\":4,\"offset\":0,\"shape\":[2]}],\"version\":1}";
  Header h{};
  std::memcpy(h.magic, magic, 8);
  h.version = 1;
  h.json_size = static_cast<uint32_t>(meta.size());
  h.data_offset = 512;
  const uint16_t values[] = {0x3F80, 0xC020};
  std::ofstream out(path, std::ios::binary);
  out.write(reinterpret_cast<const char*>(&h), sizeof h);
  out.write(meta.data(), static_cast<std::streamsize>(meta.size()));
  out.seekp(512);
  out.write(reinterpret_cast<const char*>(values), sizeof values);
}

void test_loads_bf16_tensor(const std::string& dir) {
  const std::string path = dir + "/weight.qbin";
  write_bf16_fixture(path);
  infer::ModelArchive archive(path);
  expect(archive.records().size() == 1, "one record");
  const auto& rec = archive.record("weight");
  expect(rec.dtype == infer::DType::kBFloat16, "bfloat16 dtype");
  expect(rec.shape == infer::Shape({2}), "shape [2]");
  expect(rec.nbytes == 4, "nbytes 4");
  const auto* values = static_cast<const uint16_t*>(archive.data("weight"));
  expect(values[0] == 0x3F80 && values[1] == 0xC020, "payload 0x3F80 0xC020");
  expect(archive.data_offset() == 512 && archive.mapped_bytes() == 516, "offsets");
  expect(archive.contains("weight") && !archive.contains("other"), "contains");
  bool threw = false;
  try {
    (void)archive.record("other");
  } catch (const infer::Error& e) {
    threw = std::string(e.what()) == "missing tensor: other";
  }
  expect(threw, "missing tensor throws");
}

void test_bad_magic_throws(const std::string& dir) {
  const std::string path = dir + "/bad.qbin";
  write_bf16_fixture(path, "QWENBIN2");
  bool threw = false;
  try {
    infer::ModelArchive archive(path);
  } catch (const infer::Error& e) {
    threw = std::string(e.what()) == "bad archive magic";
  }
  expect(threw, "bad magic throws");
}

// tools/export_model.py:431-522 (the W8A16 exporter self-test), through
// infer::export_archive and read back with infer::ModelArchive.
void test_w8a16_export(const std::string& dir) {
  std::vector<float> embed(20), q(210), bias = {0.125f, -0.25f, 0.5f}, norm(5), head(20);
  auto linspace = [](std::vector<float>& v, double a, double b) {
    for (size_t i = 0; i < v.size(); ++i) {
      v[i] = static_cast<float>(a + (b - a) * static_cast<double>(i) / (v.size() - 1));
    }
  };
  linspace(embed, -0.25, 0.25);
  linspace(q, -0.75, 0.75);
  for (int c = 0; c < 64; ++c) q[2 * 70 + c] = 0.0f;
  linspace(norm, 0.5, 1.5);
  linspace(head, -0.125, 0.125);
  const std::string wname = "model.layers.0.self_attn.q_proj.weight";
  const std::vector<infer::SourceTensor> src = {
      {"model.embed_tokens.weight", {4, 5}, embed.data()},
      {wname, {3, 70}, q.data()},
      {"model.layers.0.self_attn.q_proj.bias", {3}, bias.data()},
      {"model.norm.weight", {5}, norm.data()},
      {"lm_head.weight", {4, 5}, head.data()}};
  const std::string path = dir + "/model.w8a16.qbin";
  const auto report = infer::export_archive(path, src, "w8a16", 64, "cpp-test");
  expect(report.tensor_count == 6 && report.quantized_count == 1, "6 records, 1 quantised");
  expect(report.int8_count == 1 && report.bfloat16_count == 5, "1 int8, 5 bfloat16");
  expect(report.max_groupwise_abs_error <= 0.007, "max groupwise error <= 0.007");
  infer::ModelArchive archive(path);
  archive.verify();
  expect(archive.precision() == "w8a16", "precision w8a16");
  const auto& w = archive.record(wname);
  expect(w.dtype == infer::DType::kInt8, "int8 weight");
  expect(w.quant && w.quant->group_size == 64 && w.quant->axis == 1 &&
             w.quant->scale_tensor == wname + ".scale",
         "quant record");
  const auto& s = archive.record(wname + ".scale");
  expect(s.dtype == infer::DType::kBFloat16 && s.shape == infer::Shape({3, 2}), "scale [3, 2]");
  const auto* scales = static_cast<const uint16_t*>(archive.data(wname + ".scale"));
  expect(scales[4] == 0x3F80, "zero group has scale 1");
  expect(archive.data_offset() == (1u << 20), "1 MiB data offset");
  for (const auto& rec : archive.records()) expect(rec.offset % 256 == 0, "256-byte alignment");
  bool threw = false;
  try {
    (void)infer::export_archive(dir + "/g32.qbin", src, "w8a16", 32);
  } catch (const infer::Error& e) {
    threw = std::string(e.what()) == "w8a16 currently requires group size 64";
  }
  expect(threw, "group size 32 rejected");
}

void test_config(const std::string& dir) {
  const std::string path = dir + "/config.json";
  std::ofstream(path) << "{\"model_type\": \"qwen2\", \"hidden_size\": 896, "
                         "\"intermediate_size\": 4864, \"num_hidden_layers\": 24, "
                         "\"num_attention_heads\": 14, \"num_key_value_heads\": 2, "
                         "\"vocab_size\": 151936, \"max_position_embeddings\": 32768, "
                         "\"eos_token_id\": 151645, \"rms_norm_eps\": 1e-06, "
                         "\"rope_theta\": 1000000.0}";
  const auto cfg = infer::ModelConfig::load(path);
  expect(cfg.c.hidden_size == 896 && cfg.c.num_layers == 24 && cfg.c.num_kv_heads == 2 &&
             cfg.c.vocab_size == 151936 && cfg.c.eos_token_id == 151645 &&
             cfg.max_position_embeddings == 32768,
         "Qwen2.5-0.5B config");
}

}  // namespace

int main(int argc, char** argv) {
  const std::string dir = argc > 1 ? argv[1] : "/tmp";
  try {
    test_loads_bf16_tensor(dir);
    test_bad_magic_throws(dir);
    test_w8a16_export(dir);
    test_config(dir);
  } catch (const std::exception& e) {
    std::printf("FAILED: unexpected exception: %s\n", e.what());
    return 1;
  }
  if (failures) return 1;
  std::printf("PASSED\n");
  return 0;
}
