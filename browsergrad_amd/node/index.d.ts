// Type declarations of createHipRealizerBridge: the reference's
// WebGpuRealizerBridge (packages/browsergrad-kernels/src/realizer.ts:77-280)
// with handles minted by the HIP library.
export type Handle = number;
export type FusedOp = readonly [string, number, number | null];

export interface TensorPlanInput {
  readonly valueId?: number;
  readonly value_id?: number;
  readonly data?: Uint8Array;
  readonly handle?: Handle;
}

export interface HipRealizerBridge {
  upload(data: Uint8Array, shape: readonly number[], dtype: string): Handle;
  materialize(h: Handle, shape: readonly number[], dtype: string): Promise<Uint8Array>;
  release(h: Handle): void;
  matmul(a: Handle, b: Handle, m: number, k: number, n: number, dtype: string): Handle;
  fused_elementwise(inputs: readonly Handle[], ops: readonly FusedOp[], shape: readonly number[], dtype: string): Handle;
  cast(h: Handle, srcDtype: string, dstDtype: string, shape: readonly number[]): Handle;
  flash_attention(q: Handle, k: Handle, v: Handle, mask: Handle | null, b: number, h: number, sq: number,
                  sk: number, d: number, scale: number, dtype: string): Promise<Handle>;
  conv1d(input: Handle, weight: Handle, bias: Handle | null, n: number, cIn: number, lIn: number, cOut: number,
         k: number, stride: number, padding: number, dilation: number, groups: number, lOut: number,
         dtype: string): Handle;
  conv1d_backward_input(dy: Handle, weight: Handle, n: number, cIn: number, lIn: number, cOut: number, k: number,
                        stride: number, padding: number, dilation: number, groups: number, lOut: number,
                        dtype: string): Handle;
  conv1d_backward_weight(dy: Handle, input: Handle, n: number, cIn: number, lIn: number, cOut: number, k: number,
                         stride: number, padding: number, dilation: number, groups: number, lOut: number,
                         dtype: string): Handle;
  conv1d_backward_bias(dy: Handle, n: number, cOut: number, lOut: number, dtype: string): Handle;
  conv2d(input: Handle, weight: Handle, bias: Handle | null, n: number, cIn: number, h: number, w: number,
         cOut: number, kh: number, kw: number, strideH: number, strideW: number, padH: number, padW: number,
         dilationH: number, dilationW: number, groups: number, outH: number, outW: number, dtype: string): Handle;
  conv2d_backward_input(dy: Handle, weight: Handle, n: number, cIn: number, h: number, w: number, cOut: number,
                        kh: number, kw: number, strideH: number, strideW: number, padH: number, padW: number,
                        dilationH: number, dilationW: number, groups: number, outH: number, outW: number,
                        dtype: string): Handle;
  conv2d_backward_weight(dy: Handle, input: Handle, n: number, cIn: number, h: number, w: number, cOut: number,
                         kh: number, kw: number, strideH: number, strideW: number, padH: number, padW: number,
                         dilationH: number, dilationW: number, groups: number, outH: number, outW: number,
                         dtype: string): Handle;
  conv2d_backward_bias(dy: Handle, n: number, cOut: number, outH: number, outW: number, dtype: string): Handle;
  run_tensor_plan(plan: unknown, inputs: readonly TensorPlanInput[], dtype: string): Promise<Uint8Array>;
  run_tensor_plan_semantic(plan: unknown, requests: unknown, inputs: readonly TensorPlanInput[],
                           dtype: string): Promise<Uint8Array>;
  run_tensor_plan_resident(plan: unknown, inputs: readonly TensorPlanInput[], dtype: string): Handle;
  run_tensor_plan_resident_semantic(plan: unknown, requests: unknown, inputs: readonly TensorPlanInput[],
                                    dtype: string): Promise<Handle>;
  semanticTensorPlanExecutionTrace(h: Handle): Promise<unknown>;
  aliveHandleCount(): number;
  resourceSnapshot(): Record<string, unknown>;
  flushProfiles(): Promise<Record<string, unknown>>;
  close(): void;
}

export declare class KernelError extends Error {}
export declare function createHipRealizerBridge(options?: { device?: number; profiling?: boolean }): HipRealizerBridge;
export declare function version(): string;
