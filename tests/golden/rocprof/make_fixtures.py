"""Writes the synthetic rocprofv3 CSV fixtures (column layout of rocprofv3
--output-format csv) that tests/test_bench_cpu.py feeds to bench.py's
summarizers. Values are made up and chosen so the expected results are
exact: FETCH_SIZE reads half the true bytes (a 512 MiB copy reads 262144 KiB,
so the scale is 2), WRITE_SIZE is exact."""
import csv
import os

ROOT = os.path.dirname(os.path.abspath(__file__))
DK = "void llaisys::kernels::(anonymous namespace)::decodeKernel<false, 2>(llaisys::kernels::(anonymous namespace)::DecodeArgs)"
CK = "void llaisys::kernels::(anonymous namespace)::decodeCombineKernel<false>(llaisys::kernels::(anonymous namespace)::DecodeArgs)"
COPY = "__amd_rocclr_copyBuffer"


def write(path, header, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_ALL)
        w.writerow(header)
        w.writerows(rows)


def counters(path, counter, rows):
    header = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
              "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
              "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    write(path, header, [[i, i, 1, 1, 1, 1, 1, 1, name, 64, 0, 0, 0, 0, 0, counter, val, 0, 1]
                         for i, (name, val) in enumerate(rows)])


def main():
    write(f"{ROOT}/stats/run_kernel_stats.csv",
          ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"],
          [[DK, 10, 500000, 50000.0, 90.0, 48000, 52000, 1.0], [CK, 10, 55000, 5500.0, 10.0, 5000, 6000, 1.0]])
    counters(f"{ROOT}/fetch/run_counter_collection.csv", "FETCH_SIZE", [(DK, 150000.0), (DK, 150000.0), (CK, 1000.0)])
    counters(f"{ROOT}/write/run_counter_collection.csv", "WRITE_SIZE", [(DK, 2000.0), (CK, 200.0)])
    counters(f"{ROOT}/copy_fetch/run_counter_collection.csv", "FETCH_SIZE", [(COPY, 262144.0)])
    counters(f"{ROOT}/copy_write/run_counter_collection.csv", "WRITE_SIZE", [(COPY, 524288.0)])
    header = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id", "Kernel_Name",
              "Correlation_Id", "Start_Timestamp", "End_Timestamp", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
              "Accum_VGPR_Count", "SGPR_Count", "Workgroup_Size_X", "Workgroup_Size_Y", "Workgroup_Size_Z",
              "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
    rows, t, did = [], 1000, 0
    for _ in range(3):  # three decode steps: rms_norm, a library GEMM, the argmax finish
        for name, dur, grid in [("llaisys::kernels::(anonymous namespace)::rmsNormRowsKernel(unsigned short*)", 4000, 32768),
                                ("Cijk_Alik_Bljk_BBS_BH_Bias_HA_S_SAV_UserArgs_MT32x32x128_MI16x16x1_SN_LDSB1", 9000, 65536),
                                ("void llaisys::kernels::(anonymous namespace)::argmaxFinishKernel<__hip_bfloat16>(long*)", 4000, 8192)]:
            did += 1
            rows.append(["KERNEL_DISPATCH", "Agent 1", 1, 0, 1, did, 1, name, did, t, t + dur, 0, 0, 0, 0, 0, 256, 1, 1,
                         grid, 1, 1])
            t += dur + 500
    write(f"{ROOT}/trace/run_kernel_trace.csv", header, rows)


if __name__ == "__main__":
    main()
