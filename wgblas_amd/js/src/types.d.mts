// TypeScript declarations for the argument vocabulary shared by the routines.

/** Whether a routine uses an operand or its transpose. */
export type Trans = "no-transpose" | "transpose";
/** Which triangle of a symmetric or triangular matrix is referenced. */
export type Uplo = "lower" | "upper";
/** Whether the triangular or symmetric operand multiplies from the left or the right. */
export type Side = "left" | "right";
/** Whether a triangular matrix has a unit diagonal (not read) or its stored one. */
export type Diag = "unit" | "non-unit";
/** Storage order of host arrays (a GpuMatrix carries its own). */
export type Layout = "row-major" | "column-major";
/** `gpuTimeMs` is present when the device came from `init({ benchmark: true })`. */
export type Timed = { gpuTimeMs?: number };
