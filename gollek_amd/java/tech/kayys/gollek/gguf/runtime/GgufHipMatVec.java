package tech.kayys.gollek.gguf.runtime;

import tech.kayys.gollek.gguf.loader.GGUFModel;
import tech.kayys.gollek.gguf.loader.GGUFTensorInfo;

import java.lang.foreign.Arena;
import java.lang.foreign.FunctionDescriptor;
import java.lang.foreign.Linker;
import java.lang.foreign.MemorySegment;
import java.lang.foreign.SymbolLookup;
import java.lang.foreign.ValueLayout;
import java.lang.invoke.MethodHandle;
import java.nio.charset.StandardCharsets;
import java.nio.file.Files;
import java.nio.file.Path;
import java.util.IdentityHashMap;
import java.util.Map;
import java.util.WeakHashMap;

/**
 * MI355X (gfx950) route of the GGUF mat-vec, dot and row dequantization
 * through libgollek_hip.so, the C ABI of include/gollek_hip.h, bound with the
 * FFM API the way the CLI binds its native bridge
 * (ui/gollek-cli/src/main/java/tech/kayys/gollek/cli/commands/GgufFastRun.java:1915-1990:
 * System.load, SymbolLookup.libraryLookup, Linker.downcallHandle).
 *
 * <p>Hooks (this class is package-private in the runtime package, next to
 * GgufMatVec and GgufTensorData):</p>
 * <ul>
 * <li>GgufMatVec.rows (RT/GgufMatVec.java:55-96), after the row-count and
 * output-length checks and before the prepared and raw routes:
 * <pre>
 * if (GgufHipMatVec.tryRows(model, tensor, rows, columns, layout.rowBytes(), vector, output, rowCount)) {
 *     return;
 * }
 * </pre></li>
 * <li>A prefill that runs matVecRows once per prompt token (RT/GgufTensorOps.java:666-674):
 * {@code tryMatVecBatch} with the tokens' vectors, one GEMM per weight.</li>
 * <li>GgufTensorOps.dotRow and dequantizeRow (RT/GgufTensorOps.java:636-650),
 * after checkLayoutRow: {@code tryDotRow} / {@code tryDequantizeRow}, falling
 * through to the Java code when they return false.</li>
 * <li>GgufTensorOps.clearPreparedMatrixCaches, which JavaNativeGgufBackend.close
 * calls (core/plugin/gollek-plugin-runner-gguf/.../JavaNativeGgufBackend.java:139-143):
 * {@code GgufHipMatVec.release(model)}.</li>
 * <li>A GGUF MoE layer (stacked ffn_gate_exps / ffn_up_exps / ffn_down_exps
 * and, where present, the ffn_*_shexp shared expert): {@code tryMoeLayer} in
 * place of the router probabilities, selectTopK, the per-(token, route)
 * expert loop and the shared expert of MoeForwardPass
 * (runner/safetensor/gollek-safetensor-engine/src/main/java/tech/kayys/gollek/
 * safetensor/engine/generation/moe/MoeForwardPass.java:174-247).</li>
 * </ul>
 *
 * <p>The route is taken when the system property gollek.hip.enabled is not
 * "false", the library (gollek.hip.library, default libgollek_hip.so on the
 * library path) loads with ABI major 1, gollek_hip_init accepts device
 * gollek.hip.device (default 0), and the tensor's ggml type is one the
 * library multiplies (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K).  Otherwise the try
 * methods return false and the Java routes run unchanged.  A tensor's bytes
 * (GgufTensorData.tensorData, a slice of the model's mapped segment) are
 * copied to the device once, at its first use, its prepared mat-vec layout
 * is built then unless gollek.hip.prepare is "false" (the reference's
 * auto_prepare at model load, core/plugin/gollek-plugin-runner-gguf/.../
 * JavaNativeGgufBackend.java:157-180), and
 * the device handle lives until release(model).</p>
 *
 * <p>A prepared tensor is then compacted (gollek_hip_weight_compact) unless
 * gollek.hip.compact is "false": its GGUF copy is freed and the prepared
 * layout is the one device copy, which serves every call this class makes
 * (mat-vec, row prefixes, dotRow, dequantizeRow) with the same results.  A
 * prepared layout that is not compacted is a second device copy.  Like the
 * reference's prepared caches (RT/GgufPreparedCachePolicy.java:29-42) such
 * copies are admitted under a byte budget, gollek.hip.prepare.max_bytes
 * (default: no limit; the tensor's whole size is charged when prepare is
 * asked for).  When an upload finds the device full, every such copy is
 * freed (the handles then read the GGUF bytes, with the same results),
 * preparing stops for the rest of the process, and the upload is tried once
 * more; a prepare that finds no memory only stops preparing.</p>
 *
 * <p>Status codes map back to the exceptions the Java route throws
 * (RT/GgufMatVec.java:32-35, 65-71, 196-200; RT/GgufRowDot.java:77-82;
 * GC/core/GgmlType.java:70-81): NULL to NullPointerException, ARG to
 * IllegalArgumentException, UNSUPPORTED to UnsupportedOperationException;
 * DEVICE and NOMEM, which have no Java counterpart, to
 * IllegalStateException.  The library's message is the exception's.</p>
 */
final class GgufHipMatVec {
    static final int OK = 0;
    static final int ERR_NULL = -1;
    static final int ERR_ARG = -2;
    static final int ERR_UNSUPPORTED = -3;
    static final int ERR_DEVICE = -4;
    static final int ERR_NOMEM = -5;
    static final int ROUTER_SOFTMAX = 0;
    static final int ROUTER_SIGMOID = 1;

    private static final int ABI_MAJOR = 1;
    private static final int ERR_LEN = 512;

    /** Device handles per model and tensor (GGUFTensorInfo is a record over an array: identity keys). */
    private static final Map<GGUFModel, Map<GGUFTensorInfo, MemorySegment>> HANDLES = new WeakHashMap<>();
    /** Handles holding a prepared copy, with the bytes charged for it (guarded by HANDLES). */
    private static final Map<MemorySegment, Long> PREPARED = new IdentityHashMap<>();
    /** Compacted handles: their prepared layout is their only copy (guarded by HANDLES). */
    private static final Map<MemorySegment, Boolean> COMPACTED = new IdentityHashMap<>();
    private static long preparedBytes;
    private static boolean preparingStopped;

    private GgufHipMatVec() {
    }

    static boolean supportsType(int typeId) {
        return typeId == 2 || typeId == 8 || typeId == 12 || typeId == 13 || typeId == 14;
    }

    /** output[r] = row r of the tensor . vector for r < rowCount; false when the route is not taken. */
    static boolean tryRows(GGUFModel model, GGUFTensorInfo tensor, long rows, int columns, long rowBytes,
                           float[] vector, float[] output, int rowCount) {
        Binding b = Binding.get();
        if (b == null || !supportsType(tensor.typeId())) {
            return false;
        }
        MemorySegment w = handle(b, model, tensor, rows, columns, rowBytes);
        try (Arena arena = Arena.ofConfined()) {
            MemorySegment err = arena.allocate(ERR_LEN);
            int rc = b.matvecRows(w, MemorySegment.ofArray(vector), (long) vector.length,
                    MemorySegment.ofArray(output), (long) output.length, (long) rowCount, err, (long) ERR_LEN);
            check(rc, err);
        }
        return true;
    }

    /**
     * The prefill form of matVecRows: out[t * rows + r] = row r of the tensor
     * . xRows[t * columns, (t + 1) * columns) for t < m and r < rows, i.e. the
     * m matVecRows calls the reference makes per prompt
     * (RT/GgufTensorOps.java:666-674) as one small-M GEMM on the matrix cores
     * (gollek_hip_gemm_bf16), X rounded to bf16 (nearest, ties to even) as
     * that GEMM takes it.  A tensor first seen here keeps its GGUF rows (no
     * prepared copy); one already compacted by a mat-vec holds only its
     * mat-vec layout, which serves up to four vectors of at most 4096
     * columns or two of at most 16384 (the rows then equal its mat-vecs bit
     * for bit), so past that
     * this returns false and the caller runs the m mat-vecs.  False also
     * when the route is not taken.
     */
    static boolean tryMatVecBatch(GGUFModel model, GGUFTensorInfo tensor, long rows, int columns, long rowBytes,
                                  float[] xRows, int m, float[] out) {
        Binding b = Binding.get();
        if (b == null || !supportsType(tensor.typeId())) {
            return false;
        }
        if (m < 0 || (long) xRows.length < (long) m * columns || (long) out.length < (long) m * rows) {
            throw new IllegalArgumentException("Batch of " + m + " vectors needs " + ((long) m * columns)
                    + " inputs and " + ((long) m * rows) + " outputs");
        }
        MemorySegment w = handle(b, model, tensor, rows, columns, rowBytes, false);
        synchronized (HANDLES) {
            // a compacted handle keeps the mat-vec layout only, which the GEMM
            // reads for up to four vectors of at most 4096 columns (two of at
            // most 16384)
            if (COMPACTED.containsKey(w) && (m > (columns > 4096 ? 2 : 4) || columns > 16384)) {
                return false;
            }
        }
        if (m == 0) {
            return true;
        }
        short[] x = new short[Math.multiplyExact(m, columns)];
        for (int i = 0; i < x.length; i++) {
            x[i] = bf16(xRows[i]);
        }
        try (Arena arena = Arena.ofConfined()) {
            MemorySegment err = arena.allocate(ERR_LEN);
            int rc = b.gemmBf16(w, MemorySegment.ofArray(x), (long) x.length, (long) m, MemorySegment.ofArray(out),
                    (long) out.length, err, (long) ERR_LEN);
            check(rc, err);
        }
        return true;
    }

    /** The bf16 bit pattern nearest to v (ties to even); a NaN stays a (quiet) NaN. */
    static short bf16(float v) {
        int bits = Float.floatToRawIntBits(v);
        if ((bits & 0x7FFFFFFF) > 0x7F800000) {
            return (short) ((bits >>> 16) | 0x0040);
        }
        return (short) ((bits + 0x7FFF + ((bits >>> 16) & 1)) >>> 16);
    }

    /** Row {@code row} of the tensor . vector into out[0]; false when the route is not taken. */
    static boolean tryDotRow(GGUFModel model, GGUFTensorInfo tensor, long rows, int columns, long rowBytes,
                             long row, float[] vector, float[] out) {
        Binding b = Binding.get();
        if (b == null || !supportsType(tensor.typeId())) {
            return false;
        }
        MemorySegment w = handle(b, model, tensor, rows, columns, rowBytes);
        try (Arena arena = Arena.ofConfined()) {
            MemorySegment err = arena.allocate(ERR_LEN);
            int rc = b.dotRow(w, row, MemorySegment.ofArray(vector), (long) vector.length,
                    MemorySegment.ofArray(out), err, (long) ERR_LEN);
            check(rc, err);
        }
        return true;
    }

    /** Row {@code row} dequantized into dst[0, columns), bit-exact with GgufRowDequantizer. */
    static boolean tryDequantizeRow(GGUFModel model, GGUFTensorInfo tensor, long rows, int columns, long rowBytes,
                                    long row, float[] dst) {
        Binding b = Binding.get();
        if (b == null || !supportsType(tensor.typeId())) {
            return false;
        }
        MemorySegment w = handle(b, model, tensor, rows, columns, rowBytes);
        try (Arena arena = Arena.ofConfined()) {
            MemorySegment err = arena.allocate(ERR_LEN);
            int rc = b.dequantizeRows(w, row, 1L, MemorySegment.ofArray(dst), (long) dst.length, err,
                    (long) ERR_LEN);
            check(rc, err);
        }
        return true;
    }

    /**
     * One MoE layer's experts for {@code tokens} tokens: the router on
     * {@code logits} (row-major tokens x nExperts, the router linear's output)
     * with the reference's scoring (sigmoid when the model type contains
     * "qwen" or "moe", softmax otherwise; MoeForwardPass.java:174-197), the
     * top-{@code topK} routes (selectTopK, :286-306), the routed SwiGLU experts
     * summed in route order (:217-240) into {@code out} (row-major tokens x
     * hidden), then, when sharedGate / sharedUp / sharedDown are non-null, the
     * shared expert added per token (:240-247), scaled by sigmoid(x_t .
     * sharedGateRow) when that row (the shared_expert_gate weight, hidden
     * floats) is non-null.  Experts are stacked as GGUF files store them:
     * gate and up of shape {hidden, inter, nExperts}, down {inter, hidden,
     * nExperts}; the shared expert's {hidden, sharedInter} and {sharedInter,
     * hidden}.  They stay in their GGUF layout on the device (no prepared
     * copy).  False when the route is not taken.
     */
    static boolean tryMoeLayer(GGUFModel model, GGUFTensorInfo gate, GGUFTensorInfo up, GGUFTensorInfo down,
                               int nExperts, float[] x, int tokens, float[] logits, int topK, String modelType,
                               GGUFTensorInfo sharedGate, GGUFTensorInfo sharedUp, GGUFTensorInfo sharedDown,
                               float[] sharedGateRow, float[] out) {
        Binding b = Binding.get();
        boolean shared = sharedGate != null && sharedUp != null && sharedDown != null;
        if (b == null || !supportsType(gate.typeId()) || !supportsType(up.typeId()) || !supportsType(down.typeId())
                || (shared && (!supportsType(sharedGate.typeId()) || !supportsType(sharedUp.typeId())
                        || !supportsType(sharedDown.typeId())))) {
            return false;
        }
        // The library reads x, logits and the gate row by these lengths.
        long hidden = gate.shape()[0];
        if (tokens < 0 || (long) x.length < (long) tokens * hidden
                || (long) logits.length < (long) tokens * (long) nExperts
                || (sharedGateRow != null && (long) sharedGateRow.length < hidden)) {
            throw new IllegalArgumentException("MoE layer inputs are shorter than tokens x hidden / experts");
        }
        String mt = modelType != null ? modelType : "";
        int scoring = mt.contains("qwen") || mt.contains("moe") ? ROUTER_SIGMOID : ROUTER_SOFTMAX;
        MemorySegment g = expertHandle(b, model, gate);
        MemorySegment u = expertHandle(b, model, up);
        MemorySegment d = expertHandle(b, model, down);
        try (Arena arena = Arena.ofConfined()) {
            MemorySegment err = arena.allocate(ERR_LEN);
            int rc = b.moeBlock(g, u, d, (long) nExperts, MemorySegment.ofArray(x), (long) tokens,
                    MemorySegment.ofArray(logits), (long) topK, scoring, MemorySegment.ofArray(out), (long) out.length,
                    err, (long) ERR_LEN);
            check(rc, err);
            if (shared) {
                MemorySegment row = sharedGateRow != null ? MemorySegment.ofArray(sharedGateRow) : MemorySegment.NULL;
                rc = b.moeSharedExpert(expertHandle(b, model, sharedGate), expertHandle(b, model, sharedUp),
                        expertHandle(b, model, sharedDown), row, MemorySegment.ofArray(x), (long) tokens,
                        MemorySegment.ofArray(out), (long) out.length, err, (long) ERR_LEN);
                check(rc, err);
            }
        }
        return true;
    }

    /** An expert tensor's handle: rows = the product of its outer dimensions, the GGUF bytes as stored. */
    private static MemorySegment expertHandle(Binding b, GGUFModel model, GGUFTensorInfo tensor) {
        long[] shape = tensor.shape();
        long rows = 1L;
        for (int i = 1; i < shape.length; i++) {
            rows *= shape[i];
        }
        return handle(b, model, tensor, rows, Math.toIntExact(shape[0]), tensor.sizeInBytes() / rows, false);
    }

    /** Frees every device handle of the model (the prepared-cache clear). */
    static void release(GGUFModel model) {
        Binding b = Binding.get();
        Map<GGUFTensorInfo, MemorySegment> handles;
        synchronized (HANDLES) {
            handles = HANDLES.remove(model);
            if (handles != null) {
                for (MemorySegment w : handles.values()) {
                    COMPACTED.remove(w);
                    Long charged = PREPARED.remove(w);
                    if (charged != null) {
                        preparedBytes -= charged.longValue();
                    }
                }
            }
        }
        if (b == null || handles == null) {
            return;
        }
        for (MemorySegment w : handles.values()) {
            b.weightFree(w);
        }
    }

    private static MemorySegment handle(Binding b, GGUFModel model, GGUFTensorInfo tensor, long rows, int columns,
                                        long rowBytes) {
        return handle(b, model, tensor, rows, columns, rowBytes, true);
    }

    private static MemorySegment handle(Binding b, GGUFModel model, GGUFTensorInfo tensor, long rows, int columns,
                                        long rowBytes, boolean prepare) {
        synchronized (HANDLES) {
            Map<GGUFTensorInfo, MemorySegment> perModel = HANDLES.computeIfAbsent(model, m -> new IdentityHashMap<>());
            MemorySegment w = perModel.get(tensor);
            if (w != null) {
                return w;
            }
            MemorySegment bytes = GgufTensorData.tensorData(model, tensor);
            try (Arena arena = Arena.ofConfined()) {
                MemorySegment err = arena.allocate(ERR_LEN);
                w = b.weightUpload(tensor.typeId(), bytes, rows, (long) columns, rowBytes, err, (long) ERR_LEN);
                if (w.address() == 0L && b.lastStatus() == ERR_NOMEM && dropPreparedCopies(b, err)) {
                    // Earlier tensors' prepared copies filled the device: their memory is back.
                    w = b.weightUpload(tensor.typeId(), bytes, rows, (long) columns, rowBytes, err, (long) ERR_LEN);
                }
                if (w.address() == 0L) {
                    check(b.lastStatus(), err);
                    throw new IllegalStateException("gollek_hip_weight_upload returned no handle");
                }
                // The prepared mat-vec layout, built once like the reference's prepared
                // matrices (gollek.gguf.java_native.auto_prepare) within the byte budget;
                // without it the handle keeps reading the GGUF bytes.
                long size = rows * rowBytes;
                if (prepare && !preparingStopped && !"false".equals(System.getProperty("gollek.hip.prepare", "true"))
                        && preparedBytes <= Long.getLong("gollek.hip.prepare.max_bytes", Long.MAX_VALUE) - size) {
                    int rc = b.weightPrepare(w, err, (long) ERR_LEN);
                    if (rc == OK) {
                        // one copy when compacted; otherwise a second one, charged
                        boolean compacted = !"false".equals(System.getProperty("gollek.hip.compact", "true"))
                                && b.weightCompact(w, err, (long) ERR_LEN) == OK;
                        if (compacted) {
                            COMPACTED.put(w, Boolean.TRUE);
                        } else {
                            PREPARED.put(w, size);
                            preparedBytes += size;
                        }
                    } else if (rc == ERR_NOMEM) {
                        preparingStopped = true;
                    } else {
                        b.weightFree(w);
                        check(rc, err);
                    }
                }
            }
            perModel.put(tensor, w);
            return w;
        }
    }

    /** Frees every prepared copy (caller holds HANDLES) and stops preparing; false when there was none. */
    private static boolean dropPreparedCopies(Binding b, MemorySegment err) {
        preparingStopped = true;
        if (PREPARED.isEmpty()) {
            return false;
        }
        for (MemorySegment w : PREPARED.keySet()) {
            check(b.weightUnprepare(w, err, (long) ERR_LEN), err);
        }
        PREPARED.clear();
        preparedBytes = 0L;
        return true;
    }

    private static void check(int rc, MemorySegment err) {
        if (rc == OK) {
            return;
        }
        String message = err.getString(0L, StandardCharsets.UTF_8);
        switch (rc) {
            case ERR_NULL -> throw new NullPointerException(message);
            case ERR_ARG -> throw new IllegalArgumentException(message);
            case ERR_UNSUPPORTED -> throw new UnsupportedOperationException(message);
            default -> throw new IllegalStateException(message);
        }
    }

    /** The library's downcall handles, one per exported function this class uses. */
    static final class Binding {
        private static final Object LOCK = new Object();
        private static volatile Binding instance;
        private static volatile boolean unavailable;

        private final MethodHandle version;
        private final MethodHandle init;
        private final MethodHandle lastStatus;
        private final MethodHandle weightUpload;
        private final MethodHandle weightFree;
        private final MethodHandle weightPrepare;
        private final MethodHandle weightUnprepare;
        private final MethodHandle weightCompact;
        private final MethodHandle matvecRows;
        private final MethodHandle dotRow;
        private final MethodHandle dequantizeRows;
        private final MethodHandle moeBlock;
        private final MethodHandle moeSharedExpert;
        private final MethodHandle gemmBf16;

        /** The binding, or null when the route is disabled or the library cannot be used here. */
        static Binding get() {
            Binding b = instance;
            if (b != null || unavailable) {
                return b;
            }
            synchronized (LOCK) {
                if (instance == null && !unavailable) {
                    try {
                        if ("false".equals(System.getProperty("gollek.hip.enabled", "true"))) {
                            unavailable = true;
                        } else {
                            instance = new Binding(libraryPath(), Integer.getInteger("gollek.hip.device", 0).intValue());
                        }
                    } catch (Throwable t) {
                        unavailable = true;  // no library, no device or a mismatched ABI: stay on the Java routes
                    }
                }
                return instance;
            }
        }

        private static Path libraryPath() {
            String configured = System.getProperty("gollek.hip.library");
            if (configured != null && !configured.isBlank()) {
                return Path.of(configured);
            }
            for (String dir : System.getProperty("java.library.path", "").split(java.io.File.pathSeparator)) {
                if (!dir.isBlank()) {
                    Path candidate = Path.of(dir, System.mapLibraryName("gollek_hip"));
                    if (Files.isRegularFile(candidate)) {
                        return candidate;
                    }
                }
            }
            return Path.of(System.mapLibraryName("gollek_hip"));
        }

        private Binding(Path library, int device) throws Throwable {
            System.load(library.toAbsolutePath().toString());
            Linker linker = Linker.nativeLinker();
            SymbolLookup lookup = SymbolLookup.libraryLookup(library, Arena.global());
            this.version = downcall(linker, lookup, "gollek_hip_version",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT), false);
            this.init = downcall(linker, lookup, "gollek_hip_init",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.JAVA_INT, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG), false);
            this.lastStatus = downcall(linker, lookup, "gollek_hip_last_status",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT), false);
            this.weightUpload = downcall(linker, lookup, "gollek_hip_weight_upload",
                    FunctionDescriptor.of(ValueLayout.ADDRESS,
                            ValueLayout.JAVA_INT, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG, ValueLayout.JAVA_LONG,
                            ValueLayout.JAVA_LONG, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG), false);
            this.weightFree = downcall(linker, lookup, "gollek_hip_weight_free",
                    FunctionDescriptor.ofVoid(ValueLayout.ADDRESS), false);
            this.weightPrepare = downcall(linker, lookup, "gollek_hip_weight_prepare",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG), false);
            this.weightUnprepare = downcall(linker, lookup, "gollek_hip_weight_unprepare",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG), false);
            this.weightCompact = downcall(linker, lookup, "gollek_hip_weight_compact",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG), false);
            // The float[] arguments are passed as heap segments: critical downcalls with heap access.
            this.matvecRows = downcall(linker, lookup, "gollek_hip_matvec_rows",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG, ValueLayout.ADDRESS,
                            ValueLayout.JAVA_LONG, ValueLayout.JAVA_LONG, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG),
                    true);
            this.dotRow = downcall(linker, lookup, "gollek_hip_dot_row",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.ADDRESS, ValueLayout.JAVA_LONG, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG,
                            ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG), true);
            this.dequantizeRows = downcall(linker, lookup, "gollek_hip_dequantize_rows",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.ADDRESS, ValueLayout.JAVA_LONG, ValueLayout.JAVA_LONG, ValueLayout.ADDRESS,
                            ValueLayout.JAVA_LONG, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG), true);
            this.moeBlock = downcall(linker, lookup, "gollek_hip_moe_block",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG,
                            ValueLayout.ADDRESS, ValueLayout.JAVA_LONG, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG,
                            ValueLayout.JAVA_INT, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG, ValueLayout.ADDRESS,
                            ValueLayout.JAVA_LONG), true);
            this.moeSharedExpert = downcall(linker, lookup, "gollek_hip_moe_shared_expert",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.ADDRESS,
                            ValueLayout.ADDRESS, ValueLayout.JAVA_LONG, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG,
                            ValueLayout.ADDRESS, ValueLayout.JAVA_LONG), true);
            this.gemmBf16 = downcall(linker, lookup, "gollek_hip_gemm_bf16",
                    FunctionDescriptor.of(ValueLayout.JAVA_INT,
                            ValueLayout.ADDRESS, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG, ValueLayout.JAVA_LONG,
                            ValueLayout.ADDRESS, ValueLayout.JAVA_LONG, ValueLayout.ADDRESS, ValueLayout.JAVA_LONG),
                    true);
            int abi = (int) version.invokeExact();
            if (abi / 10000 != ABI_MAJOR) {
                throw new IllegalStateException("libgollek_hip ABI " + abi + " is not major " + ABI_MAJOR);
            }
            try (Arena arena = Arena.ofConfined()) {
                MemorySegment err = arena.allocate(ERR_LEN);
                int rc = (int) init.invokeExact(device, err, (long) ERR_LEN);
                if (rc != OK) {
                    throw new IllegalStateException(err.getString(0L, StandardCharsets.UTF_8));
                }
            }
        }

        private static MethodHandle downcall(Linker linker, SymbolLookup lookup, String name,
                                             FunctionDescriptor descriptor, boolean heapArguments) {
            MemorySegment symbol = lookup.find(name).orElseThrow(
                    () -> new IllegalStateException("libgollek_hip does not export " + name));
            return heapArguments
                    ? linker.downcallHandle(symbol, descriptor, Linker.Option.critical(true))
                    : linker.downcallHandle(symbol, descriptor);
        }

        // Typed entry points: their primitive parameters match the descriptors
        // exactly, as invokeExact requires (no boxing, no widening).

        int lastStatus() {
            try {
                return (int) lastStatus.invokeExact();
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        MemorySegment weightUpload(int typeId, MemorySegment hostBytes, long rows, long cols, long rowBytes,
                                   MemorySegment err, long errLen) {
            try {
                return (MemorySegment) weightUpload.invokeExact(typeId, hostBytes, rows, cols, rowBytes, err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        void weightFree(MemorySegment weight) {
            try {
                weightFree.invokeExact(weight);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        int weightPrepare(MemorySegment weight, MemorySegment err, long errLen) {
            try {
                return (int) weightPrepare.invokeExact(weight, err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        int weightUnprepare(MemorySegment weight, MemorySegment err, long errLen) {
            try {
                return (int) weightUnprepare.invokeExact(weight, err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        int weightCompact(MemorySegment weight, MemorySegment err, long errLen) {
            try {
                return (int) weightCompact.invokeExact(weight, err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        int matvecRows(MemorySegment weight, MemorySegment x, long xLen, MemorySegment y, long yLen, long rowCount,
                       MemorySegment err, long errLen) {
            try {
                return (int) matvecRows.invokeExact(weight, x, xLen, y, yLen, rowCount, err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        int dotRow(MemorySegment weight, long row, MemorySegment x, long xLen, MemorySegment out, MemorySegment err,
                   long errLen) {
            try {
                return (int) dotRow.invokeExact(weight, row, x, xLen, out, err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        int dequantizeRows(MemorySegment weight, long row0, long nrows, MemorySegment dst, long dstLen,
                           MemorySegment err, long errLen) {
            try {
                return (int) dequantizeRows.invokeExact(weight, row0, nrows, dst, dstLen, err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        int moeBlock(MemorySegment gate, MemorySegment up, MemorySegment down, long nExperts, MemorySegment x,
                     long tokens, MemorySegment logits, long topK, int scoring, MemorySegment out, long outLen,
                     MemorySegment err, long errLen) {
            try {
                return (int) moeBlock.invokeExact(gate, up, down, nExperts, x, tokens, logits, topK, scoring, out, outLen,
                        err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        int moeSharedExpert(MemorySegment gate, MemorySegment up, MemorySegment down, MemorySegment gateRow,
                            MemorySegment x, long tokens, MemorySegment out, long outLen, MemorySegment err,
                            long errLen) {
            try {
                return (int) moeSharedExpert.invokeExact(gate, up, down, gateRow, x, tokens, out, outLen, err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        int gemmBf16(MemorySegment weight, MemorySegment x, long xLen, long m, MemorySegment y, long yLen,
                     MemorySegment err, long errLen) {
            try {
                return (int) gemmBf16.invokeExact(weight, x, xLen, m, y, yLen, err, errLen);
            } catch (Throwable t) {
                throw propagate(t);
            }
        }

        private static RuntimeException propagate(Throwable t) {
            if (t instanceof RuntimeException r) {
                return r;
            }
            if (t instanceof Error e) {
                throw e;
            }
            return new IllegalStateException(t);
        }
    }
}
