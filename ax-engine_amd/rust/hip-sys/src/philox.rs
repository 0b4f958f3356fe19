//! Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11): the counter-based
//! generator the device uses, here for host callers that key a request's
//! uniform by its id rather than its position in the batch.  Counter
//! (row, step_lo, step_hi, purpose), key (seed_lo, seed_hi), uniform =
//! (word >> 8) * 2^-24.

const M0: u32 = 0xD251_1F53;
const M1: u32 = 0xCD9E_8D57;
const W0: u32 = 0x9E37_79B9;
const W1: u32 = 0xBB67_AE85;

pub fn philox4x32_10(mut c: [u32; 4], key: [u32; 2]) -> [u32; 4] {
    let (mut k0, mut k1) = (key[0], key[1]);
    for round in 0..10 {
        if round > 0 {
            k0 = k0.wrapping_add(W0);
            k1 = k1.wrapping_add(W1);
        }
        let p0 = u64::from(M0) * u64::from(c[0]);
        let p1 = u64::from(M1) * u64::from(c[2]);
        c = [
            ((p1 >> 32) as u32) ^ c[1] ^ k0,
            p1 as u32,
            ((p0 >> 32) as u32) ^ c[3] ^ k1,
            p0 as u32,
        ];
    }
    c
}

/// The uniform in [0, 1) of (seed, row, step), purpose 0, word 0.
pub fn philox_uniform(seed: u64, row: u32, step: u64) -> f32 {
    let w = philox4x32_10([row, step as u32, (step >> 32) as u32, 0], [seed as u32, (seed >> 32) as u32]);
    (w[0] >> 8) as f32 * (1.0 / 16_777_216.0)
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn random123_known_answer() {
        let out = philox4x32_10(
            [0x243F_6A88, 0x85A3_08D3, 0x1319_8A2E, 0x0370_7344],
            [0xA409_3822, 0x299F_31D0],
        );
        assert_eq!(out, [0xD16C_FE09, 0x94FD_CCEB, 0x5001_E420, 0x2412_6EA1]);
    }
}
