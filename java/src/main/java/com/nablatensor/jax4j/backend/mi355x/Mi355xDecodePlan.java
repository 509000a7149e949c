package com.nablatensor.jax4j.backend.mi355x;

import java.lang.foreign.MemorySegment;
import java.lang.ref.Cleaner;
import java.util.List;
import java.util.Queue;
import java.util.concurrent.ConcurrentLinkedQueue;
import java.util.concurrent.atomic.AtomicBoolean;

/**
 * A decode step built once (j4q_decode_plan_create) and replayed as one captured HIP graph:
 * per layer qkv = [q|k|v].h, h' = o.x_o + h, gate_up = [gate|up].h', h = down.x_down + h',
 * then logits = head.h, each GEMV a QuantizedOps.quantMatvec / quantMatvecAdd
 * (spi/QuantizedOps.java:27-30). Engine-local: the SPI has no decode-step object.
 *
 * <p>The plan holds strong references to every matrix it was built from, so their Cleaners
 * cannot enqueue a release while a replay may still read them (the engine also refuses to
 * release a matrix a live plan reads). {@link #close()} destroys the plan; an unreachable plan
 * is destroyed on the backend's next call, before any queued buffer release.
 */
public final class Mi355xDecodePlan implements AutoCloseable {
  private static final Cleaner CLEANER = Cleaner.create();
  private static final Queue<Long> PENDING = new ConcurrentLinkedQueue<>();

  private static final class State implements Runnable {
    final long handle;
    final AtomicBoolean closed = new AtomicBoolean();

    State(long handle) {
      this.handle = handle;
    }

    @Override
    public void run() {
      if (closed.compareAndSet(false, true)) PENDING.add(handle);
    }
  }

  private final long handle;
  @SuppressWarnings({"unused", "FieldCanBeLocal"})
  private final List<Mi355xBuffer> matrices;  // kept reachable while the plan lives
  private final State state;
  private final Cleaner.Cleanable cleanable;

  Mi355xDecodePlan(long handle, List<Mi355xBuffer> matrices) {
    this.handle = handle;
    this.matrices = List.copyOf(matrices);
    this.state = new State(handle);
    this.cleanable = CLEANER.register(this, state);
  }

  /** Enqueues one step on the engine stream; does not synchronise. */
  public void run() {
    if (state.closed.get()) throw new IllegalStateException("decode plan is closed");
    Mi355xNative.call("decodePlanRun", Mi355xNative.PLAN_RUN, handle, MemorySegment.NULL);
  }

  /** Waits for the device, then frees the graph and the plan's own buffers; idempotent. */
  @Override
  public void close() {
    if (!state.closed.compareAndSet(false, true)) return;
    Mi355xNative.call("decodePlanDestroy", Mi355xNative.PLAN_DESTROY, handle);
    cleanable.clean();
  }

  static void drainPending() {
    for (Long h; (h = PENDING.poll()) != null; ) {
      try {
        Mi355xNative.status("decodePlanDestroy", Mi355xNative.PLAN_DESTROY, h.longValue());
      } catch (RuntimeException ignored) {
        // the library is gone: nothing to free
      }
    }
  }
}
