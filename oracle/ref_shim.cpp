// ref_shim.cpp -- C entry point onto the reference's own CPU baseline.
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with
// /root/reference/baselines/cpu_baseline.cpp (read in place, never copied)
// into oracle/_ref/libref_cpu_baseline.so by oracle/Makefile, so tests and
// bench.py's cpu_baseline leg can call the reference implementation through
// ctypes.  The declaration below restates the signature of
// baselines/cpu_baseline.cpp:16-19.
void cpu_sparse_attention_csr(int num_nodes, int feat_dim,
                              const float* Q, const float* K, const float* V,
                              const int* row_ptr, const int* col_idx,
                              float* out_mat);

extern "C" void ref_cpu_sparse_attention_csr(int num_nodes, int feat_dim,
                                             const float* Q, const float* K,
                                             const float* V, const int* row_ptr,
                                             const int* col_idx, float* out_mat)
{
    cpu_sparse_attention_csr(num_nodes, feat_dim, Q, K, V, row_ptr, col_idx, out_mat);
}
