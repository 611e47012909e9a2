// Sampling.cs -- the managed token-sampling op, a static class beside Ops
// (ArborNet.Core/Functional/Ops.cs:21) in ArborNet.Core, over libarbor_hip (ArborHip.cs).
// No member is added to ITensor: the op takes the logits tensor as an argument and reads
// its device memory in place when it lives on a ROCm device (RocmBackend, directly or
// wrapped in Tensor). Host tensors are refused: the path has no CPU fallback.
using System;
using System.Collections.Generic;
using System.Text;
using ArborNet.Core.Backends;
using ArborNet.Core.Interfaces;
using ArborNet.Core.Native.PInvoke;
using ArborNet.Core.Tensors;

namespace ArborNet.Core.Functional
{
    /// <summary>The step's parameters; a filter is off at TopK 0, TopP 1, MinP 0.</summary>
    public sealed class SamplingOptions
    {
        public float Temperature { get; set; } = 1.0f;
        public float RepetitionPenalty { get; set; } = 1.0f;
        public float FrequencyPenalty { get; set; } = 0.0f;
        public float PresencePenalty { get; set; } = 0.0f;
        public int TopK { get; set; } = 0;
        public float TopP { get; set; } = 1.0f;
        public float MinP { get; set; } = 0.0f;

        internal ArborSamplingParams ToParams(int batch, int vocab, int ldLogits)
        {
            ArborSamplingParams p = ArborHip.DefaultParams(batch, vocab);
            p.LdLogits = ldLogits;
            p.Temperature = Temperature;
            p.RepetitionPenalty = RepetitionPenalty;
            p.FrequencyPenalty = FrequencyPenalty;
            p.PresencePenalty = PresencePenalty;
            p.TopK = TopK;
            p.TopP = TopP;
            p.MinP = MinP;
            return p;
        }
    }

    public static class Sampling
    {
        [ThreadStatic] private static DeviceBuffer<byte>? _workspace;

        /// <summary>The device storage of a ROCm tensor (RocmBackend itself or wrapped in Tensor).</summary>
        internal static RocmBackend DeviceTensor(ITensor t) => t switch
        {
            RocmBackend r => r,
            Tensor w when w._backend is RocmBackend r => r,
            _ => throw new NotSupportedException(
                "Sampling runs on a ROCm device: create the logits with Device.ROCm or move them with .To(Device.ROCm)."),
        };

        /// <summary>A workspace of at least `bytes` for calls of this thread (all on the
        /// default stream, so they are ordered and may share it).</summary>
        internal static IntPtr Workspace(ulong bytes, out ulong size)
        {
            if (_workspace == null || _workspace.Bytes < bytes)
            {
                _workspace?.Dispose();
                _workspace = new DeviceBuffer<byte>((long)Math.Max(bytes, 256UL));
            }
            size = _workspace.Bytes;
            return _workspace.Pointer;
        }

        /// <summary>
        /// One token id per row of `logits` ([batch, vocab], or [batch, seq, vocab] whose last
        /// position is sampled) on a ROCm device. `history` is [batch, H] (-1 = padding),
        /// `allowMask` [batch, ceil(vocab/32)] bit words (bit t &amp; 31 of word t &gt;&gt; 5 set =
        /// allowed), `uniforms` one value in [0, 1) per row. Rows report ARBOR_ID_* sentinels
        /// instead of an id when nothing can be sampled.
        /// </summary>
        public static int[] Sample(ITensor logits, float[] uniforms, SamplingOptions? options = null,
                                   int[,]? history = null, uint[,]? allowMask = null)
        {
            options ??= new SamplingOptions();
            RocmBackend x = DeviceTensor(logits);
            int[] dims = x.Shape.Dimensions;
            if (dims.Length != 2 && dims.Length != 3)
                throw new ArgumentException("logits must be [batch, vocab] or [batch, seq, vocab]", nameof(logits));
            int batch = dims[0], vocab = dims[dims.Length - 1];
            int seq = dims.Length == 3 ? dims[1] : 1;
            long ld = (long)seq * vocab;
            if (ld > int.MaxValue) throw new ArgumentException("seq * vocab must stay below 2^31", nameof(logits));
            if (uniforms.Length != batch) throw new ArgumentException("one uniform per row", nameof(uniforms));
            ArborSamplingParams p = options.ToParams(batch, vocab, (int)ld);
            // the last position of row 0; rows are ld elements apart
            IntPtr last = x.DevicePointer + (int)(((long)seq - 1) * vocab * sizeof(float));

            using var u = DeviceBuffer<float>.From(uniforms);
            using var ids = new DeviceBuffer<int>(batch);
            DeviceBuffer<int>? h = null;
            DeviceBuffer<uint>? m = null;
            try
            {
                if (history != null)
                {
                    if (history.GetLength(0) != batch) throw new ArgumentException("history rows", nameof(history));
                    p.HistLen = history.GetLength(1);
                    h = DeviceBuffer<int>.From(Flatten(history));
                }
                if (allowMask != null)
                {
                    if (allowMask.GetLength(0) != batch) throw new ArgumentException("mask rows", nameof(allowMask));
                    p.MaskWords = allowMask.GetLength(1);
                    m = DeviceBuffer<uint>.From(Flatten(allowMask));
                }
                ulong need = (ulong)ArborHip.arbor_sample_workspace_bytes(ref p);
                if (need == 0) need = 256;  // invalid params: arbor_sample reports why
                IntPtr ws = Workspace(need, out ulong wsBytes);
                ArborHip.Check(ArborHip.arbor_sample(ref p, last, h?.Pointer ?? IntPtr.Zero, m?.Pointer ?? IntPtr.Zero,
                                                     u.Pointer, ids.Pointer, IntPtr.Zero, ws, (UIntPtr)wsBytes, IntPtr.Zero),
                               nameof(ArborHip.arbor_sample));
                return ids.Download();  // synchronises, as CudaBackend.ToArray does
            }
            finally
            {
                h?.Dispose();
                m?.Dispose();
            }
        }

        private static T[] Flatten<T>(T[,] a)
        {
            var flat = new T[a.Length];
            int k = 0;
            foreach (T v in a) flat[k++] = v;  // row-major
            return flat;
        }
    }

    /// <summary>
    /// A generation loop's per-row token history, resident on the device: a ring of HistLen
    /// ids per row (-1 = empty) and the count of ids appended to each row. Step samples the
    /// last position of the model's logits and appends the sampled ids (arbor_sample_append),
    /// so the next step's penalties count them; EmbedInto then gathers the embedding rows of
    /// the sampled ids for the next forward pass (arbor_embed), without leaving the device.
    /// </summary>
    public sealed class GenerationState : IDisposable
    {
        public int Batch { get; }
        public int HistLen { get; }
        private readonly DeviceBuffer<int> _ring, _positions, _ids;

        public GenerationState(int batch, int histLen, int[,]? prompt = null)
        {
            if (histLen <= 0 || histLen > ArborHip.ARBOR_HISTORY_MAX) throw new ArgumentOutOfRangeException(nameof(histLen));
            Batch = batch;
            HistLen = histLen;
            var ring = new int[batch * histLen];
            Array.Fill(ring, -1);
            var pos = new int[batch];
            if (prompt != null)
            {
                int plen = prompt.GetLength(1), keep = Math.Min(plen, histLen);
                for (int b = 0; b < batch; ++b)
                {
                    for (int j = 0; j < keep; ++j) ring[b * histLen + j] = prompt[b, plen - keep + j];
                    pos[b] = keep % histLen;
                }
            }
            _ring = DeviceBuffer<int>.From(ring);
            _positions = DeviceBuffer<int>.From(pos);
            _ids = new DeviceBuffer<int>(batch);
        }

        /// <summary>Device pointer of the last step's ids (int32 [Batch]).</summary>
        public IntPtr Ids => _ids.Pointer;

        public int[] Step(ITensor logits, float[] uniforms, SamplingOptions? options = null)
        {
            options ??= new SamplingOptions();
            RocmBackend x = Sampling.DeviceTensor(logits);
            int[] dims = x.Shape.Dimensions;
            int vocab = dims[dims.Length - 1], seq = dims.Length == 3 ? dims[1] : 1;
            if (dims[0] != Batch) throw new ArgumentException("batch mismatch", nameof(logits));
            long ld = (long)seq * vocab;
            if (ld > int.MaxValue) throw new ArgumentException("seq * vocab must stay below 2^31", nameof(logits));
            ArborSamplingParams p = options.ToParams(Batch, vocab, (int)ld);
            p.HistLen = HistLen;
            IntPtr last = x.DevicePointer + (int)(((long)seq - 1) * vocab * sizeof(float));
            using var u = DeviceBuffer<float>.From(uniforms);
            ulong need = (ulong)ArborHip.arbor_sample_workspace_bytes(ref p);
            IntPtr ws = Sampling.Workspace(need == 0 ? 256 : need, out ulong wsBytes);
            ArborHip.Check(ArborHip.arbor_sample_append(ref p, last, _ring.Pointer, _positions.Pointer, IntPtr.Zero,
                                                        u.Pointer, _ids.Pointer, IntPtr.Zero, ws, (UIntPtr)wsBytes,
                                                        IntPtr.Zero),
                           nameof(ArborHip.arbor_sample_append));
            return _ids.Download();
        }

        /// <summary>Rows of `table` ([vocab, width] fp32 on the device) for the last step's ids,
        /// written to `output` ([Batch, width]); sentinel ids give zero rows.</summary>
        public void EmbedInto(ITensor table, ITensor output)
        {
            RocmBackend t = Sampling.DeviceTensor(table), o = Sampling.DeviceTensor(output);
            int vocab = t.Shape.Dimensions[0], width = t.Shape.Dimensions[1];
            ArborHip.Check(ArborHip.arbor_embed(_ids.Pointer, Batch, t.DevicePointer, vocab, width,
                                                ArborHip.ARBOR_DTYPE_F32, o.DevicePointer, IntPtr.Zero),
                           nameof(ArborHip.arbor_embed));
        }

        public void Dispose()
        {
            _ring.Dispose();
            _positions.Dispose();
            _ids.Dispose();
        }
    }

    /// <summary>
    /// The id -> bytes table of a tokenizer's vocabulary on the device (CSR: offsets [vocab + 1],
    /// UTF-8 bytes), built once; Decode turns a batch of sampled ids into text with one
    /// launch instead of a scan of the vocabulary per token (the reference's Decode looks each
    /// id up with FirstOrDefault over the vocabulary, ArborNet.Data/Tokenizers.cs:191-200,
    /// :304-313). Ids missing from the vocabulary, and ids outside it, decode as the unknown
    /// token, as there.
    /// </summary>
    public sealed class TokenTable : IDisposable
    {
        public int Vocab { get; }
        public int UnkId { get; }
        private readonly DeviceBuffer<int> _offsets;
        private readonly DeviceBuffer<byte> _bytes;

        public TokenTable(IReadOnlyDictionary<string, int> vocab, string unkToken)
        {
            int n = 0;
            foreach (var kv in vocab) n = Math.Max(n, kv.Value + 1);
            // the first key of each id in enumeration order, as FirstOrDefault finds it
            var text = new string?[n];
            foreach (var kv in vocab)
                if (kv.Value >= 0 && text[kv.Value] == null) text[kv.Value] = kv.Key;
            UnkId = vocab.TryGetValue(unkToken, out int u) ? u : -1;
            var offsets = new int[n + 1];
            var blob = new List<byte>();
            for (int i = 0; i < n; ++i)
            {
                offsets[i] = blob.Count;
                blob.AddRange(Encoding.UTF8.GetBytes(text[i] ?? unkToken));
            }
            offsets[n] = blob.Count;
            Vocab = n;
            _offsets = DeviceBuffer<int>.From(offsets);
            _bytes = DeviceBuffer<byte>.From(blob.Count > 0 ? blob.ToArray() : new byte[1]);
        }

        /// <summary>The text of `count` ids already on the device (for example GenerationState.Ids).</summary>
        public string Decode(IntPtr deviceIds, int count)
        {
            using var offs = new DeviceBuffer<int>(count + 1);
            ulong cap = 64UL * (ulong)Math.Max(count, 1);
            for (int attempt = 0; attempt < 2; ++attempt)
            {
                using var outBytes = new DeviceBuffer<byte>((long)cap);
                ArborHip.Check(ArborHip.arbor_decode(deviceIds, count, _offsets.Pointer, _bytes.Pointer, Vocab,
                                                     UnkId, offs.Pointer, outBytes.Pointer, (UIntPtr)cap, IntPtr.Zero),
                               nameof(ArborHip.arbor_decode));
                int[] o = offs.Download();
                ulong total = (ulong)o[count];
                if (total <= cap)
                {
                    byte[] all = outBytes.Download();
                    return Encoding.UTF8.GetString(all, 0, (int)total);
                }
                cap = total;  // the first call reported the size: once more with room for it
            }
            throw new InvalidOperationException("arbor_decode: output did not fit");
        }

        public string Decode(int[] ids)
        {
            using var d = DeviceBuffer<int>.From(ids);
            return Decode(d.Pointer, ids.Length);
        }

        public void Dispose()
        {
            _offsets.Dispose();
            _bytes.Dispose();
        }
    }
}
