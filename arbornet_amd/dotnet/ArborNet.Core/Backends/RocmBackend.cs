// RocmBackend.cs -- an ITensor whose storage is MI355X device memory (fp32, row-major), for
// ArborNet.Core beside CpuBackend and CudaBackend. It is the tensor the ROCm branch of the
// Tensor factories returns and the one Sampling.Sample reads logits from in place.
//
// Scope: the sampling path (logits resident on the device, sampled by libarbor_hip) runs
// natively; every other ITensor operation is carried out by CpuBackend on a host copy and
// the result uploaded again, so models keep working unchanged while their layers have no
// HIP kernels. Such results are inference tensors: autograd does not cross the device
// boundary (Backward throws).
using System;
using System.Collections.Generic;
using System.Linq;
using ArborNet.Core.Devices;
using ArborNet.Core.Interfaces;
using ArborNet.Core.Native.PInvoke;
using ArborNet.Core.Tensors;

namespace ArborNet.Core.Backends
{
    public sealed class RocmBackend : ITensor, IDisposable
    {
        private IntPtr _devicePtr;
        private readonly TensorShape _shape;
        private readonly Device _device;
        private bool _disposed;

        public TensorShape Shape => _shape;
        public Device Device => _device;
        public bool RequiresGrad { get; set; }
        public ITensor? Grad { get; set; }
        public Func<ITensor, ITensor>? GradFn { get; set; }
        public float[] Data => ToArray();

        /// <summary>Device address of element 0 (row-major fp32).</summary>
        public IntPtr DevicePointer => _disposed ? throw new ObjectDisposedException(nameof(RocmBackend)) : _devicePtr;

        private RocmBackend(TensorShape shape, Device? device)
        {
            _shape = shape?.Clone() ?? throw new ArgumentNullException(nameof(shape));
            _device = device ?? Device.ROCm;
            ulong bytes = (ulong)_shape.TotalElements * sizeof(float);
            _devicePtr = ArborHip.Malloc(Math.Max(bytes, 4UL));
            GC.AddMemoryPressure((long)bytes);
        }

        // ---- factories (the ROCm branch of Tensor.Zeros / Ones / FromScalar / FromArray / Rand / Randn / Eye) ----
        public static ITensor Zeros(TensorShape shape, Device? device = null)
        {
            var t = new RocmBackend(shape, device);
            ArborHip.Check(ArborHip.arbor_memset(t._devicePtr, 0, (UIntPtr)((ulong)shape.TotalElements * sizeof(float))),
                           nameof(ArborHip.arbor_memset));
            return t;
        }

        public static ITensor FromArray(float[] data, TensorShape shape, Device? device = null)
        {
            if (data == null) throw new ArgumentNullException(nameof(data));
            if (data.Length != shape.TotalElements)
                throw new ArgumentException($"Data length ({data.Length}) must match shape total elements ({shape.TotalElements}).");
            var t = new RocmBackend(shape, device);
            t.Upload(data);
            return t;
        }

        public static ITensor Ones(TensorShape shape, Device? device = null) =>
            FromArray(Enumerable.Repeat(1.0f, shape.TotalElements).ToArray(), shape, device);

        public static ITensor FromScalar(float value, Device? device = null) =>
            FromArray(new[] { value }, new TensorShape(1), device);

        public static ITensor Rand(TensorShape shape, Device? device = null) =>
            FromArray(CpuBackend.Rand(shape, Device.CPU).ToArray(), shape, device);

        public static ITensor Randn(TensorShape shape, Device? device = null) =>
            FromArray(CpuBackend.Randn(shape, Device.CPU).ToArray(), shape, device);

        public static ITensor Eye(int n, Device? device = null) =>
            FromArray(CpuBackend.Eye(n, Device.CPU).ToArray(), new TensorShape(n, n), device);

        private unsafe void Upload(float[] data)
        {
            fixed (float* src = data)
                ArborHip.Memcpy(_devicePtr, (IntPtr)src, (ulong)data.Length * sizeof(float), ArborHip.MemcpyHostToDevice);
        }

        public unsafe float[] ToArray()
        {
            var host = new float[_shape.TotalElements];
            fixed (float* dst = host)
                ArborHip.Memcpy((IntPtr)dst, DevicePointer, (ulong)host.Length * sizeof(float), ArborHip.MemcpyDeviceToHost);
            return host;
        }

        public void SetData(float[] floats)
        {
            if (floats.Length != _shape.TotalElements) throw new ArgumentException("length mismatch", nameof(floats));
            Upload(floats);
        }

        public float ToScalar()
        {
            if (_shape.TotalElements != 1) throw new InvalidOperationException("Tensor is not a scalar.");
            return ToArray()[0];
        }

        public ITensor Clone()
        {
            var t = new RocmBackend(_shape, _device);
            ArborHip.Memcpy(t._devicePtr, DevicePointer, (ulong)_shape.TotalElements * sizeof(float), ArborHip.MemcpyDeviceToDevice);
            return t;
        }

        public ITensor To(Device device) =>
            device.Type == DeviceType.ROCm ? Clone() : Tensor.FromArray(ToArray(), _shape, device);

        public bool IsCpu() => false;
        public bool IsCuda() => false;
        public IEnumerable<ITensor> Parameters() { yield return this; }

        // ---- every other operation: CpuBackend on a host copy, the result back on the device ----
        private ITensor Host() => CpuBackend.FromArray(ToArray(), _shape, Device.CPU);
        private static ITensor HostOf(ITensor t) => t is RocmBackend r ? r.Host() : t;
        private ITensor Dev(ITensor host) => FromArray(host.ToArray(), host.Shape, _device);

        public ITensor ArgMin(int axis) => Dev(Host().ArgMin(axis));
        public ITensor ArgMax(int axis) => Dev(Host().ArgMax(axis));
        public ITensor Add(ITensor other) => Dev(Host().Add(HostOf(other)));
        public ITensor Subtract(ITensor other) => Dev(Host().Subtract(HostOf(other)));
        public ITensor Multiply(ITensor other) => Dev(Host().Multiply(HostOf(other)));
        public ITensor Divide(ITensor other) => Dev(Host().Divide(HostOf(other)));
        public ITensor Add(float scalar) => Dev(Host().Add(scalar));
        public ITensor Subtract(float scalar) => Dev(Host().Subtract(scalar));
        public ITensor Multiply(float scalar) => Dev(Host().Multiply(scalar));
        public ITensor Divide(float scalar) => Dev(Host().Divide(scalar));
        public ITensor Subtract(int other) => Dev(Host().Subtract(other));
        public ITensor Multiply(double scalar) => Dev(Host().Multiply(scalar));
        public ITensor Divide(double scalar) => Dev(Host().Divide(scalar));
        public ITensor Negate() => Dev(Host().Negate());
        public ITensor Exp() => Dev(Host().Exp());
        public ITensor Log() => Dev(Host().Log());
        public ITensor Sqrt() => Dev(Host().Sqrt());
        public ITensor Abs() => Dev(Host().Abs());
        public ITensor Sin() => Dev(Host().Sin());
        public ITensor Cos() => Dev(Host().Cos());
        public ITensor Pow(float exponent) => Dev(Host().Pow(exponent));
        public ITensor Pow(ITensor exponent) => Dev(Host().Pow(HostOf(exponent)));
        public ITensor MatMul(ITensor other) => Dev(Host().MatMul(HostOf(other)));
        public ITensor Transpose(int[] perm) => Dev(Host().Transpose(perm));
        public ITensor Reshape(params int[] newShape) => Dev(Host().Reshape(newShape));
        public ITensor Sum(int? axis = null) => Dev(Host().Sum(axis));
        public ITensor Mean(int? axis = null) => Dev(Host().Mean(axis));
        public ITensor Mean(int[] axes) => Dev(Host().Mean(axes));
        public ITensor Max(int axis = -1) => Dev(Host().Max(axis));
        public ITensor Min(int axis = -1) => Dev(Host().Min(axis));
        public ITensor Tanh() => Dev(Host().Tanh());
        public ITensor Relu() => Dev(Host().Relu());
        public ITensor Sigmoid() => Dev(Host().Sigmoid());
        public ITensor Softmax(int axis = -1) => Dev(Host().Softmax(axis));
        public ITensor Slice(params (int start, int end, int step)[] slices) => Dev(Host().Slice(slices));
        public ITensor Concat(IEnumerable<ITensor> others, int axis = 0) =>
            Dev(Host().Concat(others.Select(HostOf).ToList(), axis));
        public ITensor BroadcastTo(TensorShape targetShape) => Dev(Host().BroadcastTo(targetShape));
        public ITensor BroadcastAdd(ITensor other) => Dev(Host().BroadcastAdd(HostOf(other)));
        public ITensor ReshapeWithBroadcast(TensorShape target, int axis) => Dev(Host().ReshapeWithBroadcast(target, axis));
        public ITensor GreaterThan(ITensor other) => Dev(Host().GreaterThan(HostOf(other)));
        public ITensor GreaterThanOrEqual(ITensor other) => Dev(Host().GreaterThanOrEqual(HostOf(other)));
        public ITensor LessEqual(ITensor other) => Dev(Host().LessEqual(HostOf(other)));
        public ITensor Where(ITensor condition, ITensor trueValue, ITensor falseValue) =>
            Dev(Host().Where(HostOf(condition), HostOf(trueValue), HostOf(falseValue)));
        public ITensor Sign() => Dev(Host().Sign());
        public ITensor LogicalNot() => Dev(Host().LogicalNot());
        public ITensor Clip(float v1, float v2) => Dev(Host().Clip(v1, v2));
        public ITensor CumSum(int axis) => Dev(Host().CumSum(axis));
        public ITensor Equal(ITensor other) => Dev(Host().Equal(HostOf(other)));

        public void Backward(ITensor? gradient = null) =>
            throw new NotSupportedException("RocmBackend tensors are inference tensors: autograd stays on the CPU and CUDA backends.");

        public void ClearGrad() => Grad = null;

        public void Dispose()
        {
            if (!_disposed)
            {
                ArborHip.Free(_devicePtr);
                GC.RemoveMemoryPressure((long)_shape.TotalElements * sizeof(float));
                _devicePtr = IntPtr.Zero;
                _disposed = true;
            }
            GC.SuppressFinalize(this);
        }

        ~RocmBackend()
        {
            if (!_disposed && _devicePtr != IntPtr.Zero) ArborHip.arbor_free(_devicePtr);
        }
    }
}
