// Scalar numerics of the sparse-MoE hot path, identical on host and device.
//
// Every function reproduces the reference crate's f32 semantics bit for bit:
// bf16 rounding by integer addition (src/expert.rs:315-322), SiLU and sigmoid
// through f32::exp (src/expert.rs:562-576), and the total order used to rank
// router logits (src/router.rs:241-247). Compile with -ffp-contract=off: an
// unfused multiply followed by an add is part of the contract.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FW_HD __host__ __device__ __forceinline__

namespace fw {

FW_HD uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
FW_HD float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
FW_HD uint64_t f64_bits(double d) { return __builtin_bit_cast(uint64_t, d); }
FW_HD double bits_f64(uint64_t u) { return __builtin_bit_cast(double, u); }

// src/expert.rs:315-318: (bits + 0x7fff + lsb) >> 16, u32 wrapping, no NaN case.
FW_HD uint16_t to_bf16(float f) {
    uint32_t b = f32_bits(f);
    return (uint16_t)((b + (0x7fffu + ((b >> 16) & 1u))) >> 16);
}
// src/expert.rs:320-322.
FW_HD float from_bf16(uint32_t v) { return bits_f32((v & 0xffffu) << 16); }
// Low and high bf16 of a packed little-endian pair.
FW_HD float bf16_lo(uint32_t pair) { return bits_f32(pair << 16); }
FW_HD float bf16_hi(uint32_t pair) { return bits_f32(pair & 0xffff0000u); }

// Round-to-nearest multiply and add that the compiler may not contract.
FW_HD float mul_rn(float a, float b) { return a * b; }
FW_HD float add_rn(float a, float b) { return a + b; }

// 2^(i/32) as correctly rounded doubles, minus i << 47 in the bit pattern, so
// that adding k << 47 for k = 32m + i scales by 2^m as well.
struct Exp2Table {
    uint64_t v[32];
};

// expf by the table method published with glibc 2.27+ (ARM optimized-routines
// expf, Szabolcs Nagy): x * 32/ln2 = k + r, exp(x) = 2^(k/32) * 2^(r/32), with
// 2^(r/32) from a cubic. Restated here with the operation order that glibc's
// x86-64 FMA build evaluates (the reduction and the polynomial fused), which
// reproduces glibc 2.35 expf, and therefore Rust f32::exp on Linux, on all 2^32
// inputs (tests/test_abi_host.py, test_expf_matches_glibc_on_all_floats). The table is a constant computed
// from 2^(i/32) in fw_exp2_table().
FW_HD float expf_glibc(float x, const uint64_t* tab) {
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double kShift = 0x1.8p+52;
    const double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint32_t ux = f32_bits(x);
    uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                     // |x| >= 88 or NaN
        if (ux == 0xff800000u) return 0.0f;     // -inf
        if (abstop >= 0x7f8u) return x + x;     // +inf, NaN
        if (x > 0x1.62e42ep6f) return bits_f32(0x7f800000u);  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                  // underflow
    }
    double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    uint64_t ki = f64_bits(kd);
    kd = kd - kShift;
    double r = __builtin_fma(kInvLn2N, xd, -kd);
    uint64_t t = tab[ki & 31u] + (ki << 47);
    double s = bits_f64(t);
    double z = __builtin_fma(kC0, r, kC1);
    double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// src/expert.rs:565-569: silu = bf16(g / (1 + exp(-g))).
FW_HD uint16_t silu_bf16(uint32_t gate_bits, const uint64_t* tab) {
    float g = from_bf16(gate_bits);
    float denominator = add_rn(1.0f, expf_glibc(-g, tab));
    return to_bf16(g / denominator);
}

// src/expert.rs:562-571: bf16(silu(gate) * up).
FW_HD uint16_t swiglu_bf16(uint32_t gate_bits, uint32_t up_bits, const uint64_t* tab) {
    float silu = from_bf16(silu_bf16(gate_bits, tab));
    return to_bf16(mul_rn(silu, from_bf16(up_bits)));
}

// src/expert.rs:573-576.
FW_HD uint16_t sigmoid_bf16(uint32_t v_bits, const uint64_t* tab) {
    float v = from_bf16(v_bits);
    float denominator = add_rn(1.0f, expf_glibc(-v, tab));
    return to_bf16(1.0f / denominator);
}

// src/expert.rs:578-580.
FW_HD uint16_t add_bf16(uint32_t a, uint32_t b) { return to_bf16(add_rn(from_bf16(a), from_bf16(b))); }

// f32::total_cmp rank of a bf16 logit as an unsigned 16-bit key: larger key =
// larger logit, -0.0 below +0.0, NaNs outermost (src/router.rs:241-247).
FW_HD uint32_t total_order_key16(uint32_t bf16_bits) {
    uint32_t b = bf16_bits & 0xffffu;
    return (b & 0x8000u) ? ((~b) & 0xffffu) : (b | 0x8000u);
}

// Selection key of (logit, expert): the maximum is the larger logit, then the
// smaller expert index. Experts must be < 65536.
FW_HD uint32_t topk_key(uint32_t bf16_bits, uint32_t expert) {
    return (total_order_key16(bf16_bits) << 16) | (0xffffu - expert);
}
FW_HD uint32_t topk_key_expert(uint32_t key) { return 0xffffu - (key & 0xffffu); }

}  // namespace fw
