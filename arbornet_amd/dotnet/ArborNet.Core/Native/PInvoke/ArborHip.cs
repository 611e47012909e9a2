// ArborHip.cs -- P/Invoke binding of libarbor_hip.so (include/arbor_sampling.h), the
// MI355X token-sampling library. Goes into ArborNet.Core beside the CUDA binding it replaces
// for this path (ArborNet.Core/Native/PInvoke/CUDA.cs:90-202): every declaration below is
// an extern "C" entry point of the header, with the header's parameter order; every
// pointer but the params struct is a device pointer.
//
// tests/test_managed_binding.py parses this file and checks names, parameter order and
// types, the params struct and the constants against the header.
using System;
using System.Runtime.InteropServices;

namespace ArborNet.Core.Native.PInvoke
{
    /// <summary>arbor_sampling_params: a host POD passed by pointer (ref).</summary>
    [StructLayout(LayoutKind.Sequential)]
    public struct ArborSamplingParams
    {
        public uint StructSize;
        public int Batch;
        public int Vocab;
        public int LdLogits;
        public int Dtype;
        public float Temperature;
        public float RepetitionPenalty;
        public float FrequencyPenalty;
        public float PresencePenalty;
        public int TopK;
        public float TopP;
        public float MinP;
        public int HistLen;
        public int MaskWords;
        public uint Flags;
    }

    public static class ArborHip
    {
        // DllImport("arbor_hip") resolves to libarbor_hip.so on Linux (arbor_hip.dll on Windows)
        private const string Lib = "arbor_hip";

        public const int ARBOR_ABI_VERSION = 1;
        public const int ARBOR_DTYPE_F32 = 0;
        public const int ARBOR_DTYPE_BF16 = 1;
        public const uint ARBOR_FLAG_WRITE_PROBS = 1;
        public const int ARBOR_VOCAB_MAX = 1048575;
        public const int ARBOR_HISTORY_MAX = 4096;
        public const int ARBOR_LM_WEIGHT_HV = 0;  // [hidden, vocab]: Linear.weight (in x out)
        public const int ARBOR_LM_WEIGHT_VH = 1;  // [vocab, hidden]

        public const int ARBOR_OK = 0;
        public const int ARBOR_ERR_NULL = -1;
        public const int ARBOR_ERR_STRUCT_SIZE = -2;
        public const int ARBOR_ERR_SHAPE = -3;
        public const int ARBOR_ERR_DTYPE = -4;
        public const int ARBOR_ERR_TEMPERATURE = -5;
        public const int ARBOR_ERR_PENALTY = -6;
        public const int ARBOR_ERR_TOP_K = -7;
        public const int ARBOR_ERR_TOP_P = -8;
        public const int ARBOR_ERR_MIN_P = -9;
        public const int ARBOR_ERR_HISTORY = -10;
        public const int ARBOR_ERR_MASK = -11;
        public const int ARBOR_ERR_WORKSPACE = -12;
        public const int ARBOR_ERR_FLAGS = -13;
        public const int ARBOR_ERR_NO_DEVICE = -14;

        public const int ARBOR_ID_EMPTY = -1;
        public const int ARBOR_ID_INVALID = -2;
        public const int ARBOR_ID_BAD_HISTORY = -3;
        public const int ARBOR_ID_STALLED = -4;

        public const uint ARBOR_NOALLOC_SCRATCH_BYTES = 16u << 20;

        // memcpy kinds (hipMemcpyKind values, as CUDA.cudaMemcpyKind)
        public const int MemcpyHostToDevice = 1;
        public const int MemcpyDeviceToHost = 2;
        public const int MemcpyDeviceToDevice = 3;

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_sample(ref ArborSamplingParams p, IntPtr logits, IntPtr history,
            IntPtr allowMask, IntPtr uniforms, IntPtr outIds, IntPtr outProbs,
            IntPtr workspace, UIntPtr workspaceBytes, IntPtr stream);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_sample_append(ref ArborSamplingParams p, IntPtr logits,
            IntPtr history, IntPtr positions, IntPtr allowMask, IntPtr uniforms, IntPtr outIds,
            IntPtr outProbs, IntPtr workspace, UIntPtr workspaceBytes, IntPtr stream);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_sample_noalloc(ref ArborSamplingParams p, IntPtr logits,
            IntPtr history, IntPtr allowMask, IntPtr uniforms, IntPtr outIds, IntPtr outProbs,
            IntPtr stream);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern UIntPtr arbor_sample_workspace_bytes(ref ArborSamplingParams p);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern void arbor_sampling_params_init(out ArborSamplingParams p, int batch, int vocab);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_device_count(out int count);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_malloc(out IntPtr ptr, UIntPtr bytes);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_free(IntPtr ptr);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_memcpy(IntPtr dst, IntPtr src, UIntPtr bytes, int kind);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_memset(IntPtr ptr, int value, UIntPtr bytes);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_synchronize();

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern IntPtr arbor_last_error();

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_abi_version();

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_decode(IntPtr ids, int count, IntPtr tokenOffsets, IntPtr tokenBytes,
            int vocab, int unkId, IntPtr outOffsets, IntPtr outBytes, UIntPtr outCapacity, IntPtr stream);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_embed(IntPtr ids, int count, IntPtr table, int vocab, int width, int dtype,
            IntPtr outRows, IntPtr stream);

        // The LM head before the sampler: logits = (x . W + bias) * scale on the matrix cores,
        // the product Linear.Forward computes as input.MatMul(weight).Add(bias) (Linear.cs:29).
        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern UIntPtr arbor_lm_head_packed_bytes(int hidden, int vocab);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_lm_head_pack(IntPtr weight, int weightDtype, int layout, int hidden, int vocab,
            IntPtr packed, IntPtr stream);

        [DllImport(Lib, CallingConvention = CallingConvention.Cdecl)]
        public static extern int arbor_lm_head(IntPtr x, int xDtype, int batch, int ldX, IntPtr packed, IntPtr bias,
            int hidden, int vocab, float scale, IntPtr logits, int logitsDtype, int ldLogits, IntPtr rowMax,
            IntPtr stream);

        /// <summary>True when the library loads and sees a HIP device (CUDA.IsAvailable's role).</summary>
        public static bool IsAvailable()
        {
            try
            {
                return arbor_device_count(out int n) == ARBOR_OK && n > 0;
            }
            catch (DllNotFoundException)
            {
                return false;
            }
            catch (EntryPointNotFoundException)
            {
                return false;
            }
        }

        /// <summary>A nonzero status becomes an exception carrying the library's message, as
        /// CUDA.Check does for CudaError.</summary>
        public static void Check(int status, string method)
        {
            if (status != ARBOR_OK)
            {
                string msg = Marshal.PtrToStringAnsi(arbor_last_error()) ?? "";
                throw new InvalidOperationException($"arbor_hip error {status} in {method}: {msg}");
            }
        }

        public static ArborSamplingParams DefaultParams(int batch, int vocab)
        {
            arbor_sampling_params_init(out ArborSamplingParams p, batch, vocab);
            return p;
        }

        public static IntPtr Malloc(ulong bytes)
        {
            Check(arbor_malloc(out IntPtr p, (UIntPtr)bytes), nameof(arbor_malloc));
            return p;
        }

        public static void Free(IntPtr p)
        {
            if (p != IntPtr.Zero) Check(arbor_free(p), nameof(arbor_free));
        }

        public static void Memcpy(IntPtr dst, IntPtr src, ulong bytes, int kind)
        {
            Check(arbor_memcpy(dst, src, (UIntPtr)bytes, kind), nameof(arbor_memcpy));
        }
    }

    /// <summary>Device memory of unmanaged elements (ids, history rings, masks, uniforms,
    /// workspaces), owned like the reference's device buffers (CudaBackend.cs:43-46, freed in
    /// Dispose :437-449).</summary>
    public sealed class DeviceBuffer<T> : IDisposable where T : unmanaged
    {
        public IntPtr Pointer { get; private set; }
        public long Length { get; }
        public ulong Bytes => (ulong)Length * (ulong)Marshal.SizeOf<T>();

        public DeviceBuffer(long length)
        {
            if (length < 0) throw new ArgumentOutOfRangeException(nameof(length));
            Length = length;
            Pointer = ArborHip.Malloc(Math.Max(Bytes, 1UL));
        }

        public static DeviceBuffer<T> From(T[] host)
        {
            var b = new DeviceBuffer<T>(host.Length);
            b.Upload(host);
            return b;
        }

        public unsafe void Upload(T[] host)
        {
            if (host.Length != Length) throw new ArgumentException("length mismatch", nameof(host));
            fixed (T* src = host)
                ArborHip.Memcpy(Pointer, (IntPtr)src, Bytes, ArborHip.MemcpyHostToDevice);
        }

        public unsafe T[] Download()
        {
            var host = new T[Length];
            fixed (T* dst = host)
                ArborHip.Memcpy((IntPtr)dst, Pointer, Bytes, ArborHip.MemcpyDeviceToHost);
            return host;
        }

        public void Dispose()
        {
            if (Pointer != IntPtr.Zero)
            {
                ArborHip.Free(Pointer);
                Pointer = IntPtr.Zero;
            }
            GC.SuppressFinalize(this);
        }

        ~DeviceBuffer()
        {
            if (Pointer != IntPtr.Zero) ArborHip.arbor_free(Pointer);
        }
    }
}
