package com.nablatensor.jax4j.backend.mi355x;

import com.nablatensor.jax4j.tensor.DType;
import com.nablatensor.jax4j.tensor.Device;
import com.nablatensor.jax4j.tensor.QuantType;
import com.nablatensor.jax4j.tensor.Shape;
import com.nablatensor.jax4j.tensor.spi.DeviceBuffer;
import java.lang.ref.Cleaner;
import java.util.Queue;
import java.util.concurrent.ConcurrentLinkedQueue;
import java.util.concurrent.atomic.AtomicBoolean;

/**
 * An engine-owned buffer: a 64-bit j4q_buffer handle. Freed by {@link #release()} or, once
 * unreachable, by a Cleaner that only enqueues the handle; the queue drains on the backend's
 * next call, never on the Cleaner thread (the ownership convention of HipBuffer.java:33-61 and
 * HipRuntime.java:243-270).
 *
 * <p>A quantized matrix that a live decode plan reads is pinned by the engine: its release is
 * refused with IllegalArgumentException and the buffer stays valid. {@link Mi355xDecodePlan}
 * keeps the matrices it reads reachable until it is closed; a Cleaner-enqueued release that
 * the engine refuses stays queued until the plan that pins it is gone.
 */
final class Mi355xBuffer implements DeviceBuffer {
  private static final Cleaner CLEANER = Cleaner.create();
  private static final Queue<Long> PENDING = new ConcurrentLinkedQueue<>();

  /** The Cleaner's action: enqueue the handle unless release() already freed it. */
  private static final class State implements Runnable {
    final long handle;
    final AtomicBoolean released = new AtomicBoolean();

    State(long handle) {
      this.handle = handle;
    }

    @Override
    public void run() {
      if (released.compareAndSet(false, true)) PENDING.add(handle);
    }
  }

  final long handle;
  final QuantType quant;  // null for dense buffers
  private final Shape shape;
  private final DType dtype;
  private final Device device;
  private final State state;
  private final Cleaner.Cleanable cleanable;

  Mi355xBuffer(long handle, Shape shape, DType dtype, Device device, QuantType quant) {
    this.handle = handle;
    this.shape = shape;
    this.dtype = dtype;
    this.device = device;
    this.quant = quant;
    this.state = new State(handle);
    this.cleanable = CLEANER.register(this, state);
  }

  /** Deterministic free (ComputeBackend.release, spi/ComputeBackend.java:280); idempotent. */
  void release() {
    if (!state.released.compareAndSet(false, true)) return;
    try {
      Mi355xNative.call("release", Mi355xNative.RELEASE, handle);
    } catch (RuntimeException e) {
      state.released.set(false);  // refused (e.g. pinned by a live decode plan): still valid
      throw e;
    }
    cleanable.clean();  // the action sees `released` and enqueues nothing
  }

  /** Frees what the Cleaner enqueued; a release the engine refuses is kept for a later drain. */
  static void drainPending() {
    for (int n = PENDING.size(); n > 0; n--) {
      Long h = PENDING.poll();
      if (h == null) return;
      int st;
      try {
        st = Mi355xNative.status("release", Mi355xNative.RELEASE, h.longValue());
      } catch (RuntimeException e) {
        continue;  // the library is gone: nothing to free
      }
      if (st == Mi355xNative.EINVAL) PENDING.add(h);  // pinned by a live decode plan: retry later
    }
  }

  @Override
  public Shape shape() {
    return shape;
  }

  /** F32 for quantized buffers too: the logical type they decode to (CpuQuantBuffer.java:31). */
  @Override
  public DType dtype() {
    return dtype;
  }

  @Override
  public Device device() {
    return device;
  }
}
