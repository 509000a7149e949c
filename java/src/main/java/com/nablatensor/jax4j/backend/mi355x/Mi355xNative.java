package com.nablatensor.jax4j.backend.mi355x;

import static java.lang.foreign.ValueLayout.ADDRESS;
import static java.lang.foreign.ValueLayout.JAVA_INT;
import static java.lang.foreign.ValueLayout.JAVA_LONG;

import java.lang.foreign.Arena;
import java.lang.foreign.FunctionDescriptor;
import java.lang.foreign.Linker;
import java.lang.foreign.MemorySegment;
import java.lang.foreign.SymbolLookup;
import java.lang.invoke.MethodHandle;
import java.util.Optional;

/**
 * FFM downcalls into libjax4j_mi355x.so, one handle per C entry point of
 * include/jax4j_mi355x.h. The library is found by {@code JAX4J_MI355X_LIB} (a path) or by
 * name on the loader path, the override convention of the ROCm engine's HIP_RUNTIME_PATH
 * (jax4j-engine-rocm/.../HipRuntime.java:56-69). Needs {@code --enable-native-access}.
 */
final class Mi355xNative {
  private Mi355xNative() {}

  /** Status codes of the C ABI (enum j4q_status). */
  static final int OK = 0, EINVAL = 1, EUNSUPPORTED = 2, ENODEV = 3, EHIP = 4, ENOMEM = 5, EHANDLE = 6;
  /** Prefill GEMM variants (enum j4q_gemm_variant). */
  static final int GEMM_INT8 = 0, GEMM_BF16 = 1;
  /** Batched GEMV arithmetic (enum j4q_gemv_policy). */
  static final int GEMV_MATRIX_CORES = 0, GEMV_FP32 = 1;
  /** j4q_buffer_desc: 48 bytes; dims at 16 and 24, device_ptr at 40. */
  static final long BUFFER_DESC_BYTES = 48, DESC_DIM0 = 16, DESC_DIM1 = 24, DESC_DEVICE_PTR = 40;

  private static final Arena LIB_ARENA = Arena.ofShared();
  private static final Linker LINKER = Linker.nativeLinker();
  private static final SymbolLookup LIB = lookup();

  private static SymbolLookup lookup() {
    String path = Optional.ofNullable(System.getenv("JAX4J_MI355X_LIB"))
        .orElse(System.getProperty("jax4j.mi355x.lib", "libjax4j_mi355x.so"));
    try {
      return SymbolLookup.libraryLookup(path, LIB_ARENA);
    } catch (IllegalArgumentException e) {
      return name -> Optional.empty();  // isAvailable() then reports false, as the SPI asks
    }
  }

  private static MethodHandle fn(String name, FunctionDescriptor d) {
    return LIB.find(name).map(s -> LINKER.downcallHandle(s, d)).orElse(null);
  }

  static final MethodHandle PROBE = fn("j4q_probe", FunctionDescriptor.of(JAVA_INT));
  static final MethodHandle INIT = fn("j4q_init", FunctionDescriptor.of(JAVA_INT, JAVA_INT));
  static final MethodHandle LAST_ERROR = fn("j4q_last_error", FunctionDescriptor.of(ADDRESS));
  static final MethodHandle SYNC = fn("j4q_sync", FunctionDescriptor.of(JAVA_INT));
  static final MethodHandle UPLOAD_QUANT = fn("j4q_upload_quantized",
      FunctionDescriptor.of(JAVA_INT, JAVA_INT, ADDRESS, JAVA_LONG, JAVA_LONG, JAVA_LONG, ADDRESS));
  static final MethodHandle UPLOAD_F32 = fn("j4q_upload_f32",
      FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, ADDRESS, ADDRESS));
  static final MethodHandle UPLOAD_BF16 = fn("j4q_upload_bf16",
      FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, ADDRESS, ADDRESS));
  static final MethodHandle DOWNLOAD_F32 = fn("j4q_download_f32",
      FunctionDescriptor.of(JAVA_INT, JAVA_LONG, ADDRESS, JAVA_LONG));
  static final MethodHandle BUFFER_INFO = fn("j4q_buffer_info", FunctionDescriptor.of(JAVA_INT, JAVA_LONG, ADDRESS));
  static final MethodHandle RELEASE = fn("j4q_release", FunctionDescriptor.of(JAVA_INT, JAVA_LONG));
  static final MethodHandle MATVEC = fn("j4q_quant_matvec",
      FunctionDescriptor.of(JAVA_INT, JAVA_LONG, JAVA_LONG, ADDRESS));
  static final MethodHandle MATVEC_ADD = fn("j4q_quant_matvec_add",
      FunctionDescriptor.of(JAVA_INT, JAVA_LONG, JAVA_LONG, JAVA_LONG, ADDRESS));
  static final MethodHandle GATHER_ROW = fn("j4q_quant_gather_row",
      FunctionDescriptor.of(JAVA_INT, JAVA_LONG, JAVA_LONG, ADDRESS));
  static final MethodHandle SET_GEMV_POLICY = fn("j4q_set_gemv_policy",
      FunctionDescriptor.of(JAVA_INT, JAVA_INT, ADDRESS));
  static final MethodHandle MATMUL = fn("j4q_quant_matmul",
      FunctionDescriptor.of(JAVA_INT, JAVA_LONG, JAVA_LONG, JAVA_INT, ADDRESS));
  static final MethodHandle CONCAT_ROWS = fn("j4q_concat_rows",
      FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, ADDRESS));
  static final MethodHandle GGUF_OPEN = fn("j4q_gguf_open", FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS));
  static final MethodHandle GGUF_CLOSE = fn("j4q_gguf_close", FunctionDescriptor.of(JAVA_INT, JAVA_LONG));
  static final MethodHandle GGUF_FIND = fn("j4q_gguf_find_tensor",
      FunctionDescriptor.of(JAVA_INT, JAVA_LONG, ADDRESS, ADDRESS));
  static final MethodHandle GGUF_UPLOAD = fn("j4q_gguf_upload",
      FunctionDescriptor.of(JAVA_INT, JAVA_LONG, JAVA_LONG, ADDRESS));
  // Decode-step plan: layers as 7 handles each (q, k, v, o, gate, up, down) and io as six
  // device addresses (h, x_o, x_down, qkv, gate_up, logits): j4q_decode_layer / j4q_decode_io.
  static final MethodHandle PLAN_CREATE = fn("j4q_decode_plan_create",
      FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_LONG, JAVA_LONG, ADDRESS, ADDRESS));
  static final MethodHandle PLAN_RUN = fn("j4q_decode_plan_run", FunctionDescriptor.of(JAVA_INT, JAVA_LONG, ADDRESS));
  static final MethodHandle PLAN_DESTROY = fn("j4q_decode_plan_destroy", FunctionDescriptor.of(JAVA_INT, JAVA_LONG));

  /** Status to the reference's exception types (HipRuntime.java:129-141; CpuBackend.java:698-714). */
  static void check(int status, String op) {
    if (status == OK) return;
    String msg;
    try {
      msg = ((MemorySegment) LAST_ERROR.invoke()).reinterpret(4096).getString(0);
    } catch (Throwable t) {
      msg = op + " failed (code " + status + ")";
    }
    switch (status) {
      case EINVAL, EUNSUPPORTED, EHANDLE -> throw new IllegalArgumentException(msg);
      case ENODEV -> throw new IllegalStateException(msg);
      default -> throw new RuntimeException(msg);  // EHIP: "<op> failed: <hip message> (code N)"; ENOMEM
    }
  }

  /** Invokes a status-returning downcall and returns the status. */
  static int status(String op, MethodHandle h, Object... args) {
    if (h == null) throw new IllegalStateException("libjax4j_mi355x.so is not loaded (" + op + ")");
    try {
      return (int) h.invokeWithArguments(args);
    } catch (RuntimeException e) {
      throw e;
    } catch (Throwable t) {
      throw new RuntimeException(op + " failed: " + t, t);
    }
  }

  /** Invokes a status-returning downcall and maps a failing status to an exception. */
  static void call(String op, MethodHandle h, Object... args) {
    check(status(op, h, args), op);
  }

  /** ComputeBackend.isAvailable: never throws (the pattern of HipRuntime.java:145-158). */
  static boolean probe() {
    if (PROBE == null) return false;
    try {
      return (int) PROBE.invoke() == 1;
    } catch (Throwable t) {
      return false;
    }
  }
}
