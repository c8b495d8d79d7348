// Custom optimizer updates compiled for their program at run time.
//
// The interpreter (RunProgram in segreduce.h) pays a decode, a dispatch and
// indexed register moves per operation for every table value. Here a program
// becomes straight-line code instead: the source generated below defines
// RtcUpdate<kEpiRtc> from the program and instantiates the library's own
// SegReduce / SegFinish templates for kEpiRtc, so the kernels are those of a
// built-in optimizer with the update inlined, and every operation is the same
// ProgApply the interpreter calls (identical results). hiprtc compiles the
// source for the device's architecture, with the floating-point flags the
// library is built with, at the first call of each program and layout; the
// code objects stay loaded until the process ends.
//
// SCEMB_CUSTOM_UPDATE selects how custom programs run: "auto" (the default:
// compiled, or interpreted when hiprtc is missing or compilation fails),
// "compile" (a call fails rather than interpret) or "interpret".
#include <dlfcn.h>
#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "segreduce.h"

namespace scemb {

// The headers the kernels are compiled from, embedded at build time
// (_build/rtc_sources.cc, written by the Makefile).
extern const char kRtcSourceSegreduce[];
extern const char kRtcSourceCommon[];
extern const char kRtcSourceScemb[];

namespace {

// libhiprtc's entry points, looked up at first use: without the library,
// custom programs are interpreted. torch ships a copy of its own; whichever
// copy the process has loaded under the soname serves.
struct Hiprtc {
  decltype(&hiprtcCreateProgram) create = nullptr;
  decltype(&hiprtcAddNameExpression) add_name = nullptr;
  decltype(&hiprtcCompileProgram) compile = nullptr;
  decltype(&hiprtcGetProgramLogSize) log_size = nullptr;
  decltype(&hiprtcGetProgramLog) log = nullptr;
  decltype(&hiprtcGetCodeSize) code_size = nullptr;
  decltype(&hiprtcGetCode) code = nullptr;
  decltype(&hiprtcGetLoweredName) lowered_name = nullptr;
  decltype(&hiprtcDestroyProgram) destroy = nullptr;
  std::string error;  // why the library is unavailable
};

template <typename F>
bool Sym(void* lib, const char* name, F* f) {
  *f = reinterpret_cast<F>(dlsym(lib, name));
  return *f != nullptr;
}

const Hiprtc& GetHiprtc() {
  static const Hiprtc h = [] {
    Hiprtc r;
    void* lib = nullptr;
    for (const char* name :
         {"libhiprtc.so.7", "libhiprtc.so", "/opt/rocm/lib/libhiprtc.so"}) {
      lib = dlopen(name, RTLD_NOW | RTLD_LOCAL);
      if (lib != nullptr) break;
    }
    if (lib == nullptr) {
      r.error = "libhiprtc not found";
      return r;
    }
    if (!Sym(lib, "hiprtcCreateProgram", &r.create) ||
        !Sym(lib, "hiprtcAddNameExpression", &r.add_name) ||
        !Sym(lib, "hiprtcCompileProgram", &r.compile) ||
        !Sym(lib, "hiprtcGetProgramLogSize", &r.log_size) ||
        !Sym(lib, "hiprtcGetProgramLog", &r.log) ||
        !Sym(lib, "hiprtcGetCodeSize", &r.code_size) ||
        !Sym(lib, "hiprtcGetCode", &r.code) ||
        !Sym(lib, "hiprtcGetLoweredName", &r.lowered_name) ||
        !Sym(lib, "hiprtcDestroyProgram", &r.destroy)) {
      r.create = nullptr;
      r.error = "libhiprtc lacks an entry point";
    }
    return r;
  }();
  return h;
}

enum class Mode { kAuto, kCompile, kInterpret, kUnknown };

Mode GetMode() {
  const char* e = std::getenv("SCEMB_CUSTOM_UPDATE");
  if (e == nullptr || *e == '\0' || std::strcmp(e, "auto") == 0) {
    return Mode::kAuto;
  }
  if (std::strcmp(e, "compile") == 0) return Mode::kCompile;
  if (std::strcmp(e, "interpret") == 0) return Mode::kInterpret;
  return Mode::kUnknown;
}

// RtcUpdate<kEpiRtc> for program p: registers as the interpreter numbers
// them (gradient, table value, slot values, hyperparameters, then the rest),
// one statement per instruction.
std::string UpdateSource(const DevProgram& p) {
  std::string s =
      "template <>\n"
      "__device__ __forceinline__ float RtcUpdate<kEpiRtc>(\n"
      "    float g, float t, float& s0, float& s1, const float* h) {\n";
  char line[128];
  for (int r = 0; r < SCEMB_PROGRAM_MAX_REGISTERS; ++r) {
    std::snprintf(line, sizeof(line), "  float r%d = 0.0f;\n", r);
    s += line;
  }
  s += "  r0 = g;\n  r1 = t;\n";
  if (p.num_slots >= 1) s += "  r2 = s0;\n";
  if (p.num_slots >= 2) s += "  r3 = s1;\n";
  for (int i = 0; i < p.num_hyper; ++i) {
    std::snprintf(line, sizeof(line), "  r%d = h[%d];\n", 2 + p.num_slots + i,
                  i);
    s += line;
  }
  for (int i = 0; i < p.num_ops; ++i) {
    const uint32_t w = p.code[i];
    const int op = static_cast<int>(w & 0xffu);
    const int d = static_cast<int>((w >> 8) & 31u);
    if (op == SCEMB_OP_CONST) {
      uint32_t bits;
      std::memcpy(&bits, &p.imm[i], sizeof(bits));
      std::snprintf(line, sizeof(line),
                    "  r%d = __builtin_bit_cast(float, 0x%08xu);\n", d, bits);
    } else {
      std::snprintf(line, sizeof(line),
                    "  r%d = ProgApply<%d>(r%d, r%d, r%d);\n", d, op,
                    static_cast<int>((w >> 13) & 31u),
                    static_cast<int>((w >> 18) & 31u),
                    static_cast<int>((w >> 23) & 31u));
    }
    s += line;
  }
  const int out[3] = {static_cast<int>(p.out & 31u),
                      static_cast<int>((p.out >> 8) & 31u),
                      static_cast<int>((p.out >> 16) & 31u)};
  for (int k = 0; k < p.num_slots; ++k) {
    std::snprintf(line, sizeof(line), "  s%d = r%d;\n", k, out[1 + k]);
    s += line;
  }
  std::snprintf(line, sizeof(line), "  return r%d;\n}\n", out[0]);
  s += line;
  return s;
}

struct Entry {
  int status = 1;  // 0 compiled, 1 not compiled (error says why)
  bool retry = false;  // failed loading, not compiling: a later call retries
  RtcKernels kernels{};
  std::string error;
};

// Compiles program p for one layout on the current device (architecture
// arch) and loads the result.
Entry Compile(const DevProgram& p, const std::string& arch, int g, int vec,
              int src, int unroll, bool mapped) {
  Entry e;
  const Hiprtc& rtc = GetHiprtc();
  if (rtc.create == nullptr) {
    e.error = rtc.error;
    return e;
  }
  // hiprtc declares the fixed-width integer types in __hip_internal only.
  const std::string source =
      "using __hip_internal::int8_t;\nusing __hip_internal::uint8_t;\n"
      "using __hip_internal::int16_t;\nusing __hip_internal::uint16_t;\n"
      "using __hip_internal::int32_t;\nusing __hip_internal::uint32_t;\n"
      "using __hip_internal::int64_t;\nusing __hip_internal::uint64_t;\n"
      "#include \"segreduce.h\"\n"
      "namespace scemb {\n" + UpdateSource(p) + "}  // namespace scemb\n";
  const char* names[] = {"segreduce.h", "common.h", "../../include/scemb.h"};
  const char* texts[] = {kRtcSourceSegreduce, kRtcSourceCommon,
                         kRtcSourceScemb};
  const std::string layout = std::to_string(g) + ", " + std::to_string(vec);
  const std::string m = mapped ? "true" : "false";
  const std::string reduce_expr =
      "&scemb::SegReduce<" + layout + ", " + std::to_string(src) + ", " +
      std::to_string(kEpiRtc) + ", " + std::to_string(unroll) + ", " + m + ">";
  const std::string finish_expr = "&scemb::SegFinish<" + layout + ", " +
                                  std::to_string(kEpiRtc) + ", " + m + ">";
  hiprtcProgram prog;
  if (rtc.create(&prog, source.c_str(), "scemb_custom_update.hip", 3, texts,
                 names) != HIPRTC_SUCCESS) {
    e.error = "hiprtcCreateProgram failed";
    return e;
  }
  rtc.add_name(prog, reduce_expr.c_str());
  rtc.add_name(prog, finish_expr.c_str());
  const std::string arch_opt = "--offload-arch=" + arch;
  const char* opts[] = {arch_opt.c_str(), "-O3", "-std=c++17",
                        "-ffp-contract=off", "-fno-fast-math", "-Xclang",
                        "-target-feature", "-Xclang", "-packed-fp32-ops", "-w"};
  const int num_opts = static_cast<int>(sizeof(opts) / sizeof(opts[0]));
  std::vector<char> code;
  std::string reduce_name, finish_name;
  if (rtc.compile(prog, num_opts, opts) != HIPRTC_SUCCESS) {
    size_t n = 0;
    rtc.log_size(prog, &n);
    std::string log(n, '\0');
    if (n > 0) rtc.log(prog, &log[0]);
    e.error = "compilation failed: " + log.substr(0, 2000);
  } else {
    size_t n = 0;
    rtc.code_size(prog, &n);
    code.resize(n);
    rtc.code(prog, code.data());
    const char* lowered = nullptr;
    if (rtc.lowered_name(prog, reduce_expr.c_str(), &lowered) ==
            HIPRTC_SUCCESS && lowered != nullptr) {
      reduce_name = lowered;
    }
    if (rtc.lowered_name(prog, finish_expr.c_str(), &lowered) ==
            HIPRTC_SUCCESS && lowered != nullptr) {
      finish_name = lowered;
    }
  }
  rtc.destroy(&prog);
  if (!e.error.empty()) return e;
  if (code.empty() || reduce_name.empty() || finish_name.empty()) {
    e.error = "no code object or kernel names";
    return e;
  }
  hipModule_t module;
  hipError_t rc = hipModuleLoadData(&module, code.data());
  if (rc == hipSuccess) {
    rc = hipModuleGetFunction(&e.kernels.reduce, module, reduce_name.c_str());
  }
  if (rc == hipSuccess) {
    rc = hipModuleGetFunction(&e.kernels.finish, module, finish_name.c_str());
  }
  if (rc != hipSuccess) {
    // For example inside a stream capture that forbids it: the program
    // compiled, so a later call tries again.
    e.error = std::string("loading the code object: ") + hipGetErrorString(rc);
    e.retry = true;
    return e;
  }
  e.status = 0;
  return e;
}

}  // namespace

int RtcKernelsFor(const DevProgram& p, int g, int vec, int src, int unroll,
                  bool mapped, RtcKernels* k) {
  const Mode mode = GetMode();
  if (mode == Mode::kUnknown) {
    return Fail(SCEMB_ERR_INVALID_ARGUMENT,
                "SCEMB_CUSTOM_UPDATE must be auto, compile or interpret");
  }
  if (mode == Mode::kInterpret) return kRtcInterpret;
  int dev = 0;
  SCEMB_HIP(hipGetDevice(&dev));
  // The key: device, layout, then the program's words (the register count
  // and the transcendental flag follow from them).
  char head[96];
  std::snprintf(head, sizeof(head), "%d:%d:%d:%d:%d:%d:%d:%d:%d:%u:", dev, g,
                vec, src, unroll, mapped ? 1 : 0, p.num_ops, p.num_slots,
                p.num_hyper, p.out);
  std::string key(head);
  key.append(reinterpret_cast<const char*>(p.code),
             sizeof(p.code[0]) * static_cast<size_t>(p.num_ops));
  key.append(reinterpret_cast<const char*>(p.imm),
             sizeof(p.imm[0]) * static_cast<size_t>(p.num_ops));
  static std::mutex mu;
  static std::map<std::string, Entry>* cache = new std::map<std::string, Entry>;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache->find(key);
  if (it == cache->end()) {
    hipDeviceProp_t prop;
    SCEMB_HIP(hipGetDeviceProperties(&prop, dev));
    it = cache->emplace(key, Compile(p, prop.gcnArchName, g, vec, src, unroll,
                                     mapped)).first;
  }
  const Entry e = it->second;
  if (e.retry) cache->erase(it);
  if (e.status == 0) {
    *k = e.kernels;
    return 0;
  }
  if (mode == Mode::kCompile) {
    return Fail(SCEMB_ERR_DEVICE, "custom optimizer update not compiled: " +
                                      e.error);
  }
  return kRtcInterpret;
}

}  // namespace scemb
