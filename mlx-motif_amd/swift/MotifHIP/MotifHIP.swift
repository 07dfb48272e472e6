// Swift face of the MI355X decode-attention library (libmotif_hip.so) over
// the CMotifHIP clang module.  It mirrors the entry points of the reference's
// Swift kernel layer (swift/Sources/MotifKitMLX/MotifMetalKernels.swift:
// MotifSDPADualV.apply 544-600, MotifSDPADualVQ4.apply 726-810,
// MotifGDAPostSplit.apply 930-1008, MotifPolynorm.apply 1147-1196) with raw
// device pointers in place of MLXArray: the caller owns the HIP buffers and
// the stream.  A non-OK status is returned, never thrown, so a caller keeps
// the reference's convention of falling back to its reference path and
// counting the fallback (MotifMetalKernels.swift:562-593).

import CMotifHIP

public enum MotifHIPStatus: Int32 {
    case ok = 0
    case contract = -1
    case unsupported = -2
    case workspace = -3
    case hip = -4
    case internalError = -5
}

public enum MotifHIPDType: Int32 {
    case float16 = 0
    case bfloat16 = 1
    case float32 = 2
}

/// One packed MLX-affine triple (data uint32, scales, biases) in device memory.
public struct MotifHIPQuantizedTriple {
    public var data: UnsafeMutablePointer<UInt32>
    public var scales: UnsafeMutableRawPointer
    public var biases: UnsafeMutableRawPointer
    public init(data: UnsafeMutablePointer<UInt32>, scales: UnsafeMutableRawPointer,
                biases: UnsafeMutableRawPointer) {
        self.data = data
        self.scales = scales
        self.biases = biases
    }
}

public enum MotifHIP {
    /// Message of the last non-OK status on this thread.
    public static var lastError: String { String(cString: motif_last_error()) }

    /// Workspace bytes the split-KV attention calls need (counters first; the
    /// caller zeroes the buffer once).
    public static func workspaceBytes(batch: Int, queryHeads: Int, kvHeads: Int,
                                      queryRows: Int = 1, kvLen: Int, headDim: Int) -> Int {
        Int(motif_sdpa_workspace_bytes(Int32(batch), Int32(queryHeads), Int32(kvHeads),
                                       Int32(queryRows), Int32(kvLen), Int32(headDim)))
    }

    /// y (B, Hq, 1, 2D) = [softmax(scale q K^T) V1 || softmax(scale q K^T) V2]
    /// over rows [0, kvLen) of full-capacity (B, Hkv, cap, D) buffers.
    public static func sdpaDualV(
        queries: UnsafeRawPointer, keys: UnsafeRawPointer, value1: UnsafeRawPointer,
        value2: UnsafeRawPointer, output: UnsafeMutableRawPointer, dtype: MotifHIPDType,
        batch: Int, queryHeads: Int, kvHeads: Int, headDim: Int, kvCapacity: Int, kvLen: Int,
        scale: Float, workspace: UnsafeMutableRawPointer?, workspaceBytes: Int,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_sdpa_dual_v(queries, keys, value1, value2, output, dtype.rawValue,
                                   Int32(batch), Int32(queryHeads), Int32(kvHeads),
                                   Int32(headDim), Int32(kvCapacity), Int32(kvLen), scale,
                                   workspace, workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// Same over the packed q4/q8 cache, read directly.
    public static func sdpaDualVQuantized(
        queries: UnsafeRawPointer, keys: MotifHIPQuantizedTriple,
        value1: MotifHIPQuantizedTriple, value2: MotifHIPQuantizedTriple,
        output: UnsafeMutableRawPointer, dtype: MotifHIPDType, batch: Int, queryHeads: Int,
        kvHeads: Int, headDim: Int, kvCapacity: Int, kvLen: Int, bits: Int, groupSize: Int,
        scale: Float, workspace: UnsafeMutableRawPointer?, workspaceBytes: Int,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_sdpa_dual_v_q(queries, keys.data, keys.scales, keys.biases,
                                     value1.data, value1.scales, value1.biases,
                                     value2.data, value2.scales, value2.biases,
                                     output, dtype.rawValue, Int32(batch), Int32(queryHeads),
                                     Int32(kvHeads), Int32(headDim), Int32(kvCapacity),
                                     Int32(kvLen), Int32(bits), Int32(groupSize), scale,
                                     workspace, workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// Quantise S new rows of the four slots into rows [offset, offset+S) of
    /// the cache triples (k1, k2, v1, v2) in one dispatch.
    public static func quantizedWrite4(
        k1: UnsafeRawPointer, k2: UnsafeRawPointer, v1: UnsafeRawPointer,
        v2: UnsafeRawPointer, slots: [MotifHIPQuantizedTriple], dtype: MotifHIPDType,
        batch: Int, heads: Int, rows: Int, headDim: Int, kvCapacity: Int, offset: Int,
        bits: Int, groupSize: Int, stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        guard slots.count == 4 else { return .contract }
        var data: [UnsafeMutablePointer<UInt32>?] = slots.map { $0.data }
        var scales: [UnsafeMutableRawPointer?] = slots.map { $0.scales }
        var biases: [UnsafeMutableRawPointer?] = slots.map { $0.biases }
        let rc = data.withUnsafeMutableBufferPointer { d in
            scales.withUnsafeMutableBufferPointer { s in
                biases.withUnsafeMutableBufferPointer { b in
                    motif_quant_write4(k1, k2, v1, v2, d.baseAddress, s.baseAddress,
                                       b.baseAddress, dtype.rawValue, Int32(batch),
                                       Int32(heads), Int32(rows), Int32(headDim),
                                       Int32(kvCapacity), Int32(offset), Int32(bits),
                                       Int32(groupSize), stream)
                }
            }
        }
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// y = RMSNorm(o - lambda * n[h / gr]) * w * (1 - lambda_init); lambdaFull
    /// is a device pointer to one fp32 value.
    public static func gdaPostSplit(
        attnO: UnsafeRawPointer, attnN: UnsafeRawPointer, sublnWeight: UnsafeRawPointer,
        output: UnsafeMutableRawPointer, dtype: MotifHIPDType, batch: Int, qOrigin: Int,
        qGroups: Int, gr: Int, rows: Int, channels: Int,
        lambdaFull: UnsafePointer<Float>, oneMinusLambdaInit: Float, eps: Float,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_post_split(attnO, attnN, sublnWeight, output, dtype.rawValue,
                                      Int32(batch), Int32(qOrigin), Int32(qGroups), Int32(gr),
                                      Int32(rows), Int32(channels), lambdaFull,
                                      oneMinusLambdaInit, eps, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// Workspace bytes of one fused decode step (either cache format).
    public static func gdaDecodeWorkspaceBytes(batch: Int, kvHeads: Int, gr: Int, kvLen: Int,
                                              headDim: Int) -> Int {
        Int(motif_gda_decode_workspace_bytes(Int32(batch), Int32(kvHeads), Int32(gr),
                                             Int32(kvLen), Int32(headDim)))
    }

    /// One GDA decode-attention step of a layer: origin pass (q1: kvHeads*gr
    /// heads over k1), noise pass (q2: kvHeads heads over k2), both over v1/v2,
    /// then gda_post_split; output (B, kvHeads*gr, 1, 2D).  Replaces the three
    /// calls of the reference's decode step (MotifMLXModel.swift:433-505).
    public static func gdaDecode(
        originQueries: UnsafeRawPointer, noiseQueries: UnsafeRawPointer,
        keys1: UnsafeRawPointer, keys2: UnsafeRawPointer, value1: UnsafeRawPointer,
        value2: UnsafeRawPointer, sublnWeight: UnsafeRawPointer,
        lambdaFull: UnsafePointer<Float>, oneMinusLambdaInit: Float, eps: Float,
        output: UnsafeMutableRawPointer, dtype: MotifHIPDType, batch: Int, kvHeads: Int,
        gr: Int, headDim: Int, kvCapacity: Int, kvLen: Int, scale: Float,
        workspace: UnsafeMutableRawPointer?, workspaceBytes: Int,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_decode(originQueries, noiseQueries, keys1, keys2, value1, value2,
                                  sublnWeight, lambdaFull, oneMinusLambdaInit, eps, output,
                                  dtype.rawValue, Int32(batch), Int32(kvHeads), Int32(gr),
                                  Int32(headDim), Int32(kvCapacity), Int32(kvLen), scale,
                                  workspace, workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// Same step over the packed q4/q8 cache.
    public static func gdaDecodeQuantized(
        originQueries: UnsafeRawPointer, noiseQueries: UnsafeRawPointer,
        keys1: MotifHIPQuantizedTriple, keys2: MotifHIPQuantizedTriple,
        value1: MotifHIPQuantizedTriple, value2: MotifHIPQuantizedTriple,
        sublnWeight: UnsafeRawPointer, lambdaFull: UnsafePointer<Float>,
        oneMinusLambdaInit: Float, eps: Float, output: UnsafeMutableRawPointer,
        dtype: MotifHIPDType, batch: Int, kvHeads: Int, gr: Int, headDim: Int, kvCapacity: Int,
        kvLen: Int, bits: Int, groupSize: Int, scale: Float,
        workspace: UnsafeMutableRawPointer?, workspaceBytes: Int,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_decode_q(originQueries, noiseQueries,
                                    keys1.data, keys1.scales, keys1.biases,
                                    keys2.data, keys2.scales, keys2.biases,
                                    value1.data, value1.scales, value1.biases,
                                    value2.data, value2.scales, value2.biases,
                                    sublnWeight, lambdaFull, oneMinusLambdaInit, eps, output,
                                    dtype.rawValue, Int32(batch), Int32(kvHeads), Int32(gr),
                                    Int32(headDim), Int32(kvCapacity), Int32(kvLen),
                                    Int32(bits), Int32(groupSize), scale, workspace,
                                    workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// The decode step that first writes the token's rows (newKeys1 .. newValue2,
    /// each (B, kvHeads, 1, D)) at row kvLen - 1 of the four slots, inside the
    /// attention launch when the step is fused.  kvLen counts the new row.
    public static func gdaDecodeAppend(
        originQueries: UnsafeRawPointer, noiseQueries: UnsafeRawPointer,
        newKeys1: UnsafeRawPointer, newKeys2: UnsafeRawPointer, newValue1: UnsafeRawPointer,
        newValue2: UnsafeRawPointer, keys1: UnsafeMutableRawPointer,
        keys2: UnsafeMutableRawPointer, value1: UnsafeMutableRawPointer,
        value2: UnsafeMutableRawPointer, sublnWeight: UnsafeRawPointer,
        lambdaFull: UnsafePointer<Float>, oneMinusLambdaInit: Float, eps: Float,
        output: UnsafeMutableRawPointer, dtype: MotifHIPDType, batch: Int, kvHeads: Int,
        gr: Int, headDim: Int, kvCapacity: Int, kvLen: Int, scale: Float,
        workspace: UnsafeMutableRawPointer?, workspaceBytes: Int,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_decode_append(originQueries, noiseQueries, newKeys1, newKeys2,
                                         newValue1, newValue2, keys1, keys2, value1, value2,
                                         sublnWeight, lambdaFull, oneMinusLambdaInit, eps,
                                         output, dtype.rawValue, Int32(batch), Int32(kvHeads),
                                         Int32(gr), Int32(headDim), Int32(kvCapacity),
                                         Int32(kvLen), scale, workspace, workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// Same over the packed cache: the token's rows are quantised into row
    /// kvLen - 1 (bit-exactly as quantWrite4 stores them).
    public static func gdaDecodeQuantizedAppend(
        originQueries: UnsafeRawPointer, noiseQueries: UnsafeRawPointer,
        newKeys1: UnsafeRawPointer, newKeys2: UnsafeRawPointer, newValue1: UnsafeRawPointer,
        newValue2: UnsafeRawPointer,
        keys1: MotifHIPQuantizedTriple, keys2: MotifHIPQuantizedTriple,
        value1: MotifHIPQuantizedTriple, value2: MotifHIPQuantizedTriple,
        sublnWeight: UnsafeRawPointer, lambdaFull: UnsafePointer<Float>,
        oneMinusLambdaInit: Float, eps: Float, output: UnsafeMutableRawPointer,
        dtype: MotifHIPDType, batch: Int, kvHeads: Int, gr: Int, headDim: Int, kvCapacity: Int,
        kvLen: Int, bits: Int, groupSize: Int, scale: Float,
        workspace: UnsafeMutableRawPointer?, workspaceBytes: Int,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_decode_q_append(originQueries, noiseQueries, newKeys1, newKeys2,
                                           newValue1, newValue2,
                                           keys1.data, keys1.scales, keys1.biases,
                                           keys2.data, keys2.scales, keys2.biases,
                                           value1.data, value1.scales, value1.biases,
                                           value2.data, value2.scales, value2.biases,
                                           sublnWeight, lambdaFull, oneMinusLambdaInit, eps,
                                           output, dtype.rawValue, Int32(batch),
                                           Int32(kvHeads), Int32(gr), Int32(headDim),
                                           Int32(kvCapacity), Int32(kvLen), Int32(bits),
                                           Int32(groupSize), scale, workspace, workspaceBytes,
                                           stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// Workspace bytes of a decode step with any noise-head count (0 when
    /// kvHeads does not divide noiseHeads or noiseHeads does not divide
    /// originHeads).
    public static func gdaDecodeHeadsWorkspaceBytes(batch: Int, originHeads: Int,
                                                   noiseHeads: Int, kvHeads: Int, kvLen: Int,
                                                   headDim: Int) -> Int {
        Int(motif_gda_decode_heads_workspace_bytes(Int32(batch), Int32(originHeads),
                                                   Int32(noiseHeads), Int32(kvHeads),
                                                   Int32(kvLen), Int32(headDim)))
    }

    /// The decode step for any noise-head count: originHeads queries over k1
    /// and noiseHeads over k2 (both multiples of kvHeads), origin head h paired
    /// with noise head h / (originHeads / noiseHeads) in gda_post_split.
    /// gdaDecode is the case noiseHeads == kvHeads.  newRows: nil, or the
    /// token's (k1, k2, v1, v2) rows, written at row kvLen - 1 first.
    public static func gdaDecodeHeads(
        originQueries: UnsafeRawPointer, noiseQueries: UnsafeRawPointer,
        newRows: (UnsafeRawPointer, UnsafeRawPointer, UnsafeRawPointer, UnsafeRawPointer)?,
        keys1: UnsafeMutableRawPointer, keys2: UnsafeMutableRawPointer,
        value1: UnsafeMutableRawPointer, value2: UnsafeMutableRawPointer,
        sublnWeight: UnsafeRawPointer, lambdaFull: UnsafePointer<Float>,
        oneMinusLambdaInit: Float, eps: Float, output: UnsafeMutableRawPointer,
        dtype: MotifHIPDType, batch: Int, originHeads: Int, noiseHeads: Int, kvHeads: Int,
        headDim: Int, kvCapacity: Int, kvLen: Int, scale: Float,
        workspace: UnsafeMutableRawPointer?, workspaceBytes: Int,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_decode_heads(originQueries, noiseQueries, newRows?.0, newRows?.1,
                                        newRows?.2, newRows?.3, keys1, keys2, value1, value2,
                                        sublnWeight, lambdaFull, oneMinusLambdaInit, eps, output,
                                        dtype.rawValue, Int32(batch), Int32(originHeads),
                                        Int32(noiseHeads), Int32(kvHeads), Int32(headDim),
                                        Int32(kvCapacity), Int32(kvLen), scale, workspace,
                                        workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// Same over the packed q4/q8 cache (new rows quantised as quantWrite4
    /// stores them).
    public static func gdaDecodeQuantizedHeads(
        originQueries: UnsafeRawPointer, noiseQueries: UnsafeRawPointer,
        newRows: (UnsafeRawPointer, UnsafeRawPointer, UnsafeRawPointer, UnsafeRawPointer)?,
        keys1: MotifHIPQuantizedTriple, keys2: MotifHIPQuantizedTriple,
        value1: MotifHIPQuantizedTriple, value2: MotifHIPQuantizedTriple,
        sublnWeight: UnsafeRawPointer, lambdaFull: UnsafePointer<Float>,
        oneMinusLambdaInit: Float, eps: Float, output: UnsafeMutableRawPointer,
        dtype: MotifHIPDType, batch: Int, originHeads: Int, noiseHeads: Int, kvHeads: Int,
        headDim: Int, kvCapacity: Int, kvLen: Int, bits: Int, groupSize: Int, scale: Float,
        workspace: UnsafeMutableRawPointer?, workspaceBytes: Int,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_decode_q_heads(originQueries, noiseQueries, newRows?.0, newRows?.1,
                                          newRows?.2, newRows?.3,
                                          keys1.data, keys1.scales, keys1.biases,
                                          keys2.data, keys2.scales, keys2.biases,
                                          value1.data, value1.scales, value1.biases,
                                          value2.data, value2.scales, value2.biases,
                                          sublnWeight, lambdaFull, oneMinusLambdaInit, eps,
                                          output, dtype.rawValue, Int32(batch),
                                          Int32(originHeads), Int32(noiseHeads),
                                          Int32(kvHeads), Int32(headDim), Int32(kvCapacity),
                                          Int32(kvLen), Int32(bits), Int32(groupSize), scale,
                                          workspace, workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// The RoPE position scale of a model's rope_scaling config
    /// (MotifTypes.swift:218, read as mlx-lm's initialize_rope reads it: the
    /// type is `type`, else `ropeType`, else "default").  No config and
    /// "default" give 1, "linear" gives 1 / factor; nil for a type that is
    /// not built here or a factor that is not positive and finite, where the
    /// caller must not use these entry points (positions would be wrong).
    public static func ropePositionScale(type: String?, ropeType: String?,
                                         factor: Double?) -> Float? {
        switch type ?? ropeType ?? "default" {
        case "default":
            return 1
        case "linear":
            guard let factor, factor > 0, factor.isFinite else { return nil }
            return Float(1 / factor)
        default:
            return nil
        }
    }

    /// RoPE on q and k, the q1/q2, k1/k2, v1/v2 head split and the 4-slot
    /// write in one launch: k1..v2 rows row0 ..< row0 + seqLen of buffers of
    /// `capacity` rows (the cache, or capacity = seqLen, row0 = 0 for plain
    /// tensors), positions (pos0 + s) * positionScale (ropePositionScale).
    public static func ropeSplit4(
        qProj: UnsafeRawPointer, kProj: UnsafeRawPointer, vProj: UnsafeRawPointer,
        q1: UnsafeMutableRawPointer, q2: UnsafeMutableRawPointer,
        k1: UnsafeMutableRawPointer, k2: UnsafeMutableRawPointer,
        v1: UnsafeMutableRawPointer, v2: UnsafeMutableRawPointer, dtype: MotifHIPDType,
        batch: Int, seqLen: Int, qGroups: Int, gr: Int, kGroups: Int, kRatio: Int,
        headDim: Int, capacity: Int, row0: Int, pos0: Int, theta: Float,
        positionScale: Float = 1, originFirst: Bool, stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_rope_split4_scaled(qProj, kProj, vProj, q1, q2, k1, k2, v1, v2,
                                          dtype.rawValue, Int32(batch), Int32(seqLen),
                                          Int32(qGroups), Int32(gr), Int32(kGroups),
                                          Int32(kRatio), Int32(headDim), Int32(capacity),
                                          Int32(row0), Int32(pos0), theta, positionScale,
                                          originFirst ? 1 : 0, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// Workspace bytes of gdaPrefillFromProjections (0 when its rows are not
    /// split).
    public static func gdaPrefillWorkspaceBytes(batch: Int, seqLen: Int, qGroups: Int, gr: Int,
                                                kGroups: Int, headDim: Int, kvLen: Int) -> Int {
        return Int(motif_gda_prefill_workspace_bytes(Int32(batch), Int32(seqLen), Int32(qGroups),
                                                     Int32(gr), Int32(kGroups), Int32(headDim),
                                                     Int32(kvLen)))
    }

    /// A layer's prefill chunk from the projection outputs in one attention
    /// launch: q and k roped at positions offset + s, the chunk's rows
    /// written into the 4-slot fp cache, the origin (q1 over k1) and noise
    /// (q2 over k2) dual-V passes with the bottom-right causal mask
    /// (fp16/bf16 cache, head_dim 128; other shapes return .unsupported:
    /// compose ropeSplit4 and the multi-row sdpa calls).  positionScale: 1,
    /// or 1 / factor for a "linear" rope_scaling config
    /// (ropePositionScale); other scaling types are not built.
    public static func gdaPrefillFromProjections(
        qProj: UnsafeRawPointer, kProj: UnsafeRawPointer, vProj: UnsafeRawPointer,
        keys1: UnsafeMutableRawPointer, keys2: UnsafeMutableRawPointer,
        value1: UnsafeMutableRawPointer, value2: UnsafeMutableRawPointer,
        outputOrigin: UnsafeMutableRawPointer, outputNoise: UnsafeMutableRawPointer,
        dtype: MotifHIPDType, batch: Int, seqLen: Int, qGroups: Int, gr: Int, kGroups: Int,
        headDim: Int, kvCapacity: Int, offset: Int, scale: Float, theta: Float,
        positionScale: Float = 1, originFirst: Bool, workspace: UnsafeMutableRawPointer?,
        workspaceBytes: Int, stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_prefill_proj_scaled(qProj, kProj, vProj, keys1, keys2, value1, value2,
                                               outputOrigin, outputNoise, dtype.rawValue,
                                               Int32(batch), Int32(seqLen), Int32(qGroups),
                                               Int32(gr), Int32(kGroups), Int32(headDim),
                                               Int32(kvCapacity), Int32(offset), scale, theta,
                                               positionScale, originFirst ? 1 : 0, workspace,
                                               workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// A layer's decode attention from the projection outputs: RoPE at
    /// position kvLen - 1, the head split and the token's cache rows inside
    /// the attention launch (fp16/bf16 cache, head_dim 128; other shapes
    /// return .unsupported: compose ropeSplit4 and gdaDecode).
    /// positionScale: 1, or 1 / factor for a "linear" rope_scaling config.
    public static func gdaDecodeFromProjections(
        qProj: UnsafeRawPointer, kProj: UnsafeRawPointer, vProj: UnsafeRawPointer,
        keys1: UnsafeMutableRawPointer, keys2: UnsafeMutableRawPointer,
        value1: UnsafeMutableRawPointer, value2: UnsafeMutableRawPointer,
        sublnWeight: UnsafeRawPointer, lambdaFull: UnsafePointer<Float>,
        oneMinusLambdaInit: Float, eps: Float, output: UnsafeMutableRawPointer,
        dtype: MotifHIPDType, batch: Int, kvHeads: Int, gr: Int, headDim: Int,
        kvCapacity: Int, kvLen: Int, scale: Float, theta: Float, positionScale: Float = 1,
        originFirst: Bool, workspace: UnsafeMutableRawPointer?, workspaceBytes: Int,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_decode_proj_scaled(qProj, kProj, vProj, keys1, keys2, value1, value2,
                                              sublnWeight, lambdaFull, oneMinusLambdaInit, eps,
                                              output, dtype.rawValue, Int32(batch),
                                              Int32(kvHeads), Int32(gr), Int32(headDim),
                                              Int32(kvCapacity), Int32(kvLen), scale, theta,
                                              positionScale, originFirst ? 1 : 0, workspace,
                                              workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// The same from the projection outputs over the packed q4/q8 cache: the
    /// token's roped k rows and v rows are quantised into row kvLen - 1 of
    /// the four triples inside the attention launch (fp16 scales, head_dim
    /// 128; other shapes return .unsupported: compose ropeSplit4 and
    /// gdaDecodeQuantizedAppend, which give the same values bit for bit).
    /// positionScale: 1, or 1 / factor for a "linear" rope_scaling config.
    public static func gdaDecodeQuantizedFromProjections(
        qProj: UnsafeRawPointer, kProj: UnsafeRawPointer, vProj: UnsafeRawPointer,
        keys1: MotifHIPQuantizedTriple, keys2: MotifHIPQuantizedTriple,
        value1: MotifHIPQuantizedTriple, value2: MotifHIPQuantizedTriple,
        sublnWeight: UnsafeRawPointer, lambdaFull: UnsafePointer<Float>,
        oneMinusLambdaInit: Float, eps: Float, output: UnsafeMutableRawPointer,
        dtype: MotifHIPDType, batch: Int, kvHeads: Int, gr: Int, headDim: Int,
        kvCapacity: Int, kvLen: Int, bits: Int, groupSize: Int, scale: Float, theta: Float,
        positionScale: Float = 1, originFirst: Bool, workspace: UnsafeMutableRawPointer?,
        workspaceBytes: Int, stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_gda_decode_q_proj_scaled(qProj, kProj, vProj,
                                         keys1.data, keys1.scales, keys1.biases,
                                         keys2.data, keys2.scales, keys2.biases,
                                         value1.data, value1.scales, value1.biases,
                                         value2.data, value2.scales, value2.biases,
                                         sublnWeight, lambdaFull, oneMinusLambdaInit, eps,
                                         output, dtype.rawValue, Int32(batch), Int32(kvHeads),
                                         Int32(gr), Int32(headDim), Int32(kvCapacity),
                                         Int32(kvLen), Int32(bits), Int32(groupSize), scale,
                                         theta, positionScale, originFirst ? 1 : 0, workspace,
                                         workspaceBytes, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }

    /// PolyNorm over the last axis of x (rows, D).
    public static func polynorm(
        x: UnsafeRawPointer, weight: UnsafeRawPointer, bias: UnsafeRawPointer,
        output: UnsafeMutableRawPointer, dtype: MotifHIPDType, rows: Int, dim: Int, eps: Float,
        stream: UnsafeMutableRawPointer?
    ) -> MotifHIPStatus {
        let rc = motif_polynorm(x, weight, bias, output, dtype.rawValue, Int64(rows),
                                Int32(dim), eps, stream)
        return MotifHIPStatus(rawValue: rc) ?? .hip
    }
}
