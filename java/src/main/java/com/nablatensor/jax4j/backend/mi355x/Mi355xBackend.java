package com.nablatensor.jax4j.backend.mi355x;

import static java.lang.foreign.ValueLayout.JAVA_FLOAT;
import static java.lang.foreign.ValueLayout.JAVA_INT;
import static java.lang.foreign.ValueLayout.JAVA_LONG;
import static java.lang.foreign.ValueLayout.JAVA_SHORT;

import com.nablatensor.jax4j.tensor.ConvSpec;
import com.nablatensor.jax4j.tensor.DType;
import com.nablatensor.jax4j.tensor.Device;
import com.nablatensor.jax4j.tensor.DeviceType;
import com.nablatensor.jax4j.tensor.Op;
import com.nablatensor.jax4j.tensor.QuantType;
import com.nablatensor.jax4j.tensor.Shape;
import com.nablatensor.jax4j.tensor.spi.ComputeBackend;
import com.nablatensor.jax4j.tensor.spi.DeviceBuffer;
import com.nablatensor.jax4j.tensor.spi.QuantizedOps;
import java.lang.foreign.Arena;
import java.lang.foreign.MemorySegment;
import java.lang.invoke.MethodHandle;
import java.nio.file.Path;
import java.util.ArrayList;
import java.util.Arrays;
import java.util.EnumSet;
import java.util.List;
import java.util.Set;

/**
 * The MI355X (gfx950) GGUF quantized-matmul engine as a jax4j backend: {@link ComputeBackend}
 * plus the optional {@link QuantizedOps} capability (spi/QuantizedOps.java:19-34), over the C
 * ABI of include/jax4j_mi355x.h. Selected with {@code -Djax4j.tensor.backend=mi355x}
 * (BackendRegistry.java:63-72); found by ServiceLoader through
 * META-INF/services/com.nablatensor.jax4j.tensor.spi.ComputeBackend.
 *
 * <p>The QuantizedOps methods keep the CPU backend's contract (CpuBackend.java:688-762): x holds
 * exactly cols values, y is F32 [rows], the add of quantMatvecAdd is rounded on its own. The
 * engine's extra operations (batched GEMV, prefill GEMM, GGUF upload, the decode-step plan)
 * are public methods of this class, reached by casting the backend. Dense F32 ops are outside
 * this engine and throw UnsupportedOperationException, the reference's own convention
 * (spi/ComputeBackend.java:99-101, 158-159).
 */
public final class Mi355xBackend implements ComputeBackend, QuantizedOps {
  private boolean initialized;

  @Override
  public String name() {
    return "mi355x";  // unique: "rocm" is RocmBackend's
  }

  @Override
  public DeviceType deviceType() {
    return DeviceType.ROCM;
  }

  @Override
  public boolean isAvailable() {
    return Mi355xNative.probe();
  }

  @Override
  public int priority() {
    return 60;  // above RocmBackend's 50, below CUDA's 100
  }

  private synchronized void ensureInitialized() {
    if (!initialized) {
      Mi355xNative.call("init", Mi355xNative.INIT, 0);
      initialized = true;
    }
    drainPending();
  }

  /** Plans first, so that matrices they pinned can then be released. */
  private static void drainPending() {
    Mi355xDecodePlan.drainPending();
    Mi355xBuffer.drainPending();
  }

  private static Mi355xBuffer buf(DeviceBuffer b) {
    if (b instanceof Mi355xBuffer m) return m;
    throw new IllegalArgumentException("expected an mi355x buffer, got " + b.getClass());
  }

  private static Mi355xBuffer quant(DeviceBuffer b) {
    Mi355xBuffer m = buf(b);
    if (m.quant == null) throw new IllegalArgumentException("expected an mi355x quantized buffer");
    return m;
  }

  /** Runs an entry point whose last argument is a j4q_buffer out-parameter; returns the handle. */
  private long newHandle(String op, MethodHandle h, Object... args) {
    ensureInitialized();
    try (Arena a = Arena.ofConfined()) {
      MemorySegment out = a.allocate(JAVA_LONG);
      Object[] all = Arrays.copyOf(args, args.length + 1);
      all[args.length] = out;
      Mi355xNative.call(op, h, all);
      return out.get(JAVA_LONG, 0);
    }
  }

  /** [dims0, dims1] of an engine buffer (j4q_buffer_desc.dims). */
  private static long[] dims(long handle) {
    try (Arena a = Arena.ofConfined()) {
      MemorySegment desc = a.allocate(Mi355xNative.BUFFER_DESC_BYTES, 8);
      Mi355xNative.call("bufferInfo", Mi355xNative.BUFFER_INFO, handle, desc);
      return new long[] {desc.get(JAVA_LONG, Mi355xNative.DESC_DIM0), desc.get(JAVA_LONG, Mi355xNative.DESC_DIM1)};
    }
  }

  // ---- QuantizedOps (spi/QuantizedOps.java:19-34) -------------------------------------------

  @Override
  public Set<QuantType> supportedQuantTypes() {
    return EnumSet.of(QuantType.Q2_0, QuantType.Q4_0, QuantType.Q8_0, QuantType.Q4_K, QuantType.Q6_K);
  }

  @Override
  public DeviceBuffer uploadQuantized(MemorySegment blocks, QuantType type, Shape logicalShape, Device device) {
    if (logicalShape.rank() != 2) throw new IllegalArgumentException("uploadQuantized requires [rows, cols], got " + logicalShape);
    checkDevice(device);
    try (Arena a = Arena.ofConfined()) {
      // a heap segment cannot be passed as ADDRESS: copy it to native memory first
      MemorySegment src = blocks.isNative() ? blocks : a.allocate(blocks.byteSize(), 16).copyFrom(blocks);
      long h = newHandle("uploadQuantized", Mi355xNative.UPLOAD_QUANT, type.id(), src, src.byteSize(),
          (long) logicalShape.dim(0), (long) logicalShape.dim(1));
      return new Mi355xBuffer(h, logicalShape, DType.F32, device, type);
    }
  }

  /** y(rows) = W . x: x must hold exactly cols values, as CpuBackend.java:712 requires. */
  @Override
  public DeviceBuffer quantMatvec(DeviceBuffer weights, DeviceBuffer x) {
    Mi355xBuffer w = quant(weights);
    requireVector(w, x, "quantMatvec");
    long h = newHandle("quantMatvec", Mi355xNative.MATVEC, w.handle, buf(x).handle);
    return new Mi355xBuffer(h, Shape.of(w.shape().dim(0)), DType.F32, w.device(), null);
  }

  /** y(rows) = (W . x) + add, the add rounded separately (CpuBackend.java:728-736). */
  @Override
  public DeviceBuffer quantMatvecAdd(DeviceBuffer weights, DeviceBuffer x, DeviceBuffer add) {
    Mi355xBuffer w = quant(weights);
    requireVector(w, x, "quantMatvecAdd");
    long h = newHandle("quantMatvecAdd", Mi355xNative.MATVEC_ADD, w.handle, buf(x).handle, buf(add).handle);
    return new Mi355xBuffer(h, Shape.of(w.shape().dim(0)), DType.F32, w.device(), null);
  }

  /** One dequantized row, bit-exact; rows outside [0, rows) are rejected. */
  @Override
  public DeviceBuffer quantGatherRow(DeviceBuffer weights, int row) {
    Mi355xBuffer w = quant(weights);
    long h = newHandle("quantGatherRow", Mi355xNative.GATHER_ROW, w.handle, (long) row);
    return new Mi355xBuffer(h, Shape.of(w.shape().dim(1)), DType.F32, w.device(), null);
  }

  private static void requireVector(Mi355xBuffer w, DeviceBuffer x, String op) {
    if (w.shape().rank() != 2 || w.shape().dim(1) != x.shape().size())
      throw new IllegalArgumentException(op + " shape mismatch: " + w.shape() + " x " + x.shape());
  }

  // ---- engine-local operations (no SPI counterpart) ------------------------------------------

  /** quantMatvec of every row of x [B, cols]: y F32 [B, rows] (one pass over W per 16 rows). */
  public DeviceBuffer quantMatvecBatched(DeviceBuffer weights, DeviceBuffer x) {
    Mi355xBuffer w = quant(weights);
    requireBatch(w, x, "quantMatvecBatched");
    long h = newHandle("quantMatvecBatched", Mi355xNative.MATVEC, w.handle, buf(x).handle);
    return new Mi355xBuffer(h, Shape.of(x.shape().dim(0), w.shape().dim(0)), DType.F32, w.device(), null);
  }

  /** quantMatvecAdd of every row of x [B, cols] with add [B, rows]. */
  public DeviceBuffer quantMatvecAddBatched(DeviceBuffer weights, DeviceBuffer x, DeviceBuffer add) {
    Mi355xBuffer w = quant(weights);
    requireBatch(w, x, "quantMatvecAddBatched");
    long h = newHandle("quantMatvecAddBatched", Mi355xNative.MATVEC_ADD, w.handle, buf(x).handle, buf(add).handle);
    return new Mi355xBuffer(h, Shape.of(x.shape().dim(0), w.shape().dim(0)), DType.F32, w.device(), null);
  }

  /** Arithmetic of the batched calls above, process-wide (j4q_set_gemv_policy): false (the
   *  default) runs up to 16 batch rows per pass on the matrix cores, x as hi + lo fp16 under a
   *  power-of-two scale; true runs every row on the batch-1 kernel (fp32 x, no matrix cores),
   *  each row equal bit for bit to quantMatvec of that row. Returns the previous setting. */
  public boolean batchedGemvFp32(boolean fp32) {
    try (Arena a = Arena.ofConfined()) {
      MemorySegment prev = a.allocate(JAVA_INT);
      Mi355xNative.call("setGemvPolicy", Mi355xNative.SET_GEMV_POLICY,
          fp32 ? Mi355xNative.GEMV_FP32 : Mi355xNative.GEMV_MATRIX_CORES, prev);
      return prev.get(JAVA_INT, 0) == Mi355xNative.GEMV_FP32;
    }
  }

  private static void requireBatch(Mi355xBuffer w, DeviceBuffer x, String op) {
    if (x.shape().rank() != 2 || x.shape().dim(1) != w.shape().dim(1))
      throw new IllegalArgumentException(op + " shape mismatch: " + w.shape() + " x " + x.shape());
  }

  /** bf16 activations (raw bit patterns) for the prefill GEMM; DType has no BF16, so the
   *  buffer reports F32, the type its values decode to. */
  public DeviceBuffer uploadBf16(short[] bits, Shape shape, Device device) {
    checkDevice(device);
    if (shape.size() != bits.length) throw new IllegalArgumentException("uploadBf16: " + bits.length + " values for " + shape);
    try (Arena a = Arena.ofConfined()) {
      MemorySegment host = a.allocateFrom(JAVA_SHORT, bits);
      MemorySegment dims = a.allocateFrom(JAVA_LONG, Arrays.stream(shape.dims()).asLongStream().toArray());
      long h = newHandle("uploadBf16", Mi355xNative.UPLOAD_BF16, host, shape.rank(), dims);
      return new Mi355xBuffer(h, shape, DType.F32, device, null);
    }
  }

  /** Prefill GEMM Y F32 [M, N] = X [M, K] . W^T, X from {@link #uploadBf16}: the int8 variant
   *  (Q8_0 weights; X quantized per 32-block) or the bf16 one (Q8_0, Q4_0, Q4_K, Q6_K). */
  public DeviceBuffer quantMatmul(DeviceBuffer weights, DeviceBuffer xBf16, boolean int8) {
    Mi355xBuffer w = quant(weights);
    long h = newHandle("quantMatmul", Mi355xNative.MATMUL, w.handle, buf(xBf16).handle,
        int8 ? Mi355xNative.GEMM_INT8 : Mi355xNative.GEMM_BF16);
    return new Mi355xBuffer(h, Shape.of(xBf16.shape().dim(0), w.shape().dim(0)), DType.F32, w.device(), null);
  }

  /** One matrix holding the rows of `parts` in order (same type and cols): matrices that share
   *  their input (q/k/v, gate/up) then run as one GEMV. The parts stay valid. */
  public DeviceBuffer concatRows(List<DeviceBuffer> parts) {
    List<Mi355xBuffer> ps = parts.stream().map(Mi355xBackend::quant).toList();
    try (Arena a = Arena.ofConfined()) {
      MemorySegment hs = a.allocate(JAVA_LONG, ps.size());
      int rows = 0;
      for (int i = 0; i < ps.size(); i++) {
        hs.setAtIndex(JAVA_LONG, i, ps.get(i).handle);
        rows += ps.get(i).shape().dim(0);
      }
      long h = newHandle("concatRows", Mi355xNative.CONCAT_ROWS, hs, ps.size());
      Mi355xBuffer p0 = ps.get(0);
      return new Mi355xBuffer(h, Shape.of(rows, p0.shape().dim(1)), DType.F32, p0.device(), p0.quant);
    }
  }

  /** uploadQuantized of one tensor of a .gguf file, straight from the file's mapping. */
  public DeviceBuffer uploadFromGguf(Path file, String tensor, QuantType type, Device device) {
    checkDevice(device);
    ensureInitialized();
    try (Arena a = Arena.ofConfined()) {
      MemorySegment out = a.allocate(JAVA_LONG);
      Mi355xNative.call("ggufOpen", Mi355xNative.GGUF_OPEN, a.allocateFrom(file.toString()), out);
      long f = out.get(JAVA_LONG, 0);
      try {
        Mi355xNative.call("ggufFind", Mi355xNative.GGUF_FIND, f, a.allocateFrom(tensor), out);
        long index = out.get(JAVA_LONG, 0);
        Mi355xNative.call("ggufUpload", Mi355xNative.GGUF_UPLOAD, f, index, out);
      } finally {
        Mi355xNative.status("ggufClose", Mi355xNative.GGUF_CLOSE, f);
      }
      long h = out.get(JAVA_LONG, 0);
      long[] d = dims(h);
      return new Mi355xBuffer(h, Shape.of(Math.toIntExact(d[0]), Math.toIntExact(d[1])), DType.F32, device, type);
    }
  }

  /**
   * The quantized matmuls of a decode step over `layers` (each {q, k, v, o, gate, up, down})
   * and an optional head, replayed as one HIP graph (see {@link Mi355xDecodePlan}). io: the
   * residual h [batch, d_model] (updated in place), x_o and x_down (inputs of o and down),
   * qkv and gateUp (per-layer outputs) and logits (may be null without a head). The plan keeps
   * every matrix and io buffer reachable until it is closed.
   */
  public Mi355xDecodePlan decodePlan(List<DeviceBuffer[]> layers, DeviceBuffer head, long batch, DeviceBuffer h,
      DeviceBuffer xO, DeviceBuffer xDown, DeviceBuffer qkv, DeviceBuffer gateUp, DeviceBuffer logits) {
    List<Mi355xBuffer> keep = new ArrayList<>();
    try (Arena a = Arena.ofConfined()) {
      MemorySegment ls = a.allocate(JAVA_LONG, 7L * layers.size());
      for (int l = 0; l < layers.size(); l++) {
        DeviceBuffer[] layer = layers.get(l);
        if (layer.length != 7) throw new IllegalArgumentException("decodePlan: layer " + l + " needs 7 matrices");
        for (int j = 0; j < 7; j++) {
          Mi355xBuffer m = quant(layer[j]);
          keep.add(m);
          ls.setAtIndex(JAVA_LONG, 7L * l + j, m.handle);
        }
      }
      long headHandle = 0;
      if (head != null) {
        Mi355xBuffer hb = quant(head);
        keep.add(hb);
        headHandle = hb.handle;
      }
      DeviceBuffer[] io = {h, xO, xDown, qkv, gateUp, logits};
      long[] ptrs = new long[io.length];
      for (int i = 0; i < io.length; i++) {
        if (io[i] == null) continue;
        Mi355xBuffer b = buf(io[i]);
        keep.add(b);
        ptrs[i] = devicePointer(b);
      }
      long plan = newHandle("decodePlan", Mi355xNative.PLAN_CREATE, ls, layers.size(), headHandle, batch,
          a.allocateFrom(JAVA_LONG, ptrs));
      return new Mi355xDecodePlan(plan, keep);
    }
  }

  /** Device address of an engine buffer (j4q_buffer_desc.device_ptr). */
  public long devicePointer(DeviceBuffer b) {
    try (Arena a = Arena.ofConfined()) {
      MemorySegment desc = a.allocate(Mi355xNative.BUFFER_DESC_BYTES, 8);
      Mi355xNative.call("bufferInfo", Mi355xNative.BUFFER_INFO, buf(b).handle, desc);
      return desc.get(JAVA_LONG, Mi355xNative.DESC_DEVICE_PTR);
    }
  }

  private void checkDevice(Device device) {
    if (device != null && (device.type() != DeviceType.ROCM || device.index() != 0))
      throw new IllegalArgumentException(name() + " serves rocm:0, not " + device);
  }

  // ---- ComputeBackend data movement (spi/ComputeBackend.java:48, 87, 277, 280) -------------

  @Override
  public DeviceBuffer upload(float[] data, Shape shape, DType dtype, Device device) {
    if (dtype != DType.F32) throw new IllegalArgumentException(name() + " uploads F32 only, got " + dtype);
    checkDevice(device);
    if (shape.size() != data.length) throw new IllegalArgumentException("upload: " + data.length + " values for " + shape);
    try (Arena a = Arena.ofConfined()) {
      MemorySegment host = a.allocateFrom(JAVA_FLOAT, data);
      MemorySegment dims = a.allocateFrom(JAVA_LONG, Arrays.stream(shape.dims()).asLongStream().toArray());
      long h = newHandle("upload", Mi355xNative.UPLOAD_F32, host, shape.rank(), dims);
      return new Mi355xBuffer(h, shape, DType.F32, device == null ? Device.rocm() : device, null);
    }
  }

  /** A fresh float[] after a device sync (RocmBackend.java:476-482). */
  @Override
  public float[] download(DeviceBuffer buffer) {
    Mi355xBuffer b = buf(buffer);
    if (b.quant != null) throw new IllegalArgumentException("download of a quantized buffer: use quantGatherRow");
    float[] out = new float[Math.toIntExact(b.shape().size())];
    try (Arena a = Arena.ofConfined()) {
      MemorySegment host = a.allocate(JAVA_FLOAT, out.length);
      Mi355xNative.call("download", Mi355xNative.DOWNLOAD_F32, b.handle, host, (long) out.length);
      MemorySegment.copy(host, JAVA_FLOAT, 0, out, 0, out.length);
      return out;
    }
  }

  @Override
  public void sync() {
    Mi355xNative.call("sync", Mi355xNative.SYNC);
  }

  @Override
  public void release(DeviceBuffer buffer) {
    buf(buffer).release();
  }

  // ---- the rest of ComputeBackend (spi/ComputeBackend.java:89-97, 150-156, 194-206) --------

  private UnsupportedOperationException unsupported(String op) {
    return new UnsupportedOperationException(name() + " backend does not support " + op);
  }

  @Override
  public DeviceBuffer binary(Op op, DeviceBuffer a, DeviceBuffer b) {
    throw unsupported("binary");
  }

  @Override
  public DeviceBuffer scalar(Op op, DeviceBuffer a, double value) {
    throw unsupported("scalar");
  }

  @Override
  public DeviceBuffer unary(Op op, DeviceBuffer a) {
    throw unsupported("unary");
  }

  @Override
  public DeviceBuffer transpose(DeviceBuffer a) {
    throw unsupported("transpose");
  }

  @Override
  public DeviceBuffer matmul(DeviceBuffer a, DeviceBuffer b) {
    throw unsupported("matmul");
  }

  @Override
  public DeviceBuffer reduceSum(DeviceBuffer a) {
    throw unsupported("reduceSum");
  }

  @Override
  public DeviceBuffer reduceMax(DeviceBuffer a) {
    throw unsupported("reduceMax");
  }

  @Override
  public DeviceBuffer sumAxis0(DeviceBuffer a) {
    throw unsupported("sumAxis0");
  }

  @Override
  public DeviceBuffer conv2d(DeviceBuffer x, DeviceBuffer w, ConvSpec spec) {
    throw unsupported("conv2d");
  }

  @Override
  public DeviceBuffer conv2dGradInput(DeviceBuffer upstream, DeviceBuffer w, ConvSpec spec) {
    throw unsupported("conv2dGradInput");
  }

  @Override
  public DeviceBuffer conv2dGradWeight(DeviceBuffer x, DeviceBuffer upstream, ConvSpec spec) {
    throw unsupported("conv2dGradWeight");
  }

  @Override
  public DeviceBuffer reluBackward(DeviceBuffer upstream, DeviceBuffer input) {
    throw unsupported("reluBackward");
  }

  @Override
  public DeviceBuffer broadcastTo(DeviceBuffer a, Shape target) {
    throw unsupported("broadcastTo");
  }
}
