//! `--attention-backend mi355x`: paged decode and ragged / paged causal prefill on the
//! gfx950 kernels of `libmi355x_attn.so`, through the raw ABI of the `mi355x_sys` crate.
//!
//! Drop-in for the reference server: this file becomes `src/models/attention/mi355x.rs`, a
//! child module of `backend.rs` (so it sees the private `AttentionBackend` trait,
//! `backend.rs:262-306`), declared there with `#[cfg(has_mi355x)] mod mi355x;`. It follows
//! `FlashInferAttentionBackend` (`backend.rs:316-804`) step for step: one decode plan and one
//! prefill plan per backend, re-planned once per forward and reused by every layer; graph
//! plans registered under the block-table address and re-planned outside capture; the same
//! error strings. The only differences are the ABI (raw pointers, strides and the ATen
//! current stream instead of `at::Tensor*`) and that no output tensor is allocated by the
//! library: decode and prefill write into a tensor allocated here (or the caller's static
//! output in `forward_into`).
//!
//! The edits to `backend.rs` that wire it in are listed in the repository's integration
//! guide (new `AttentionBackendKind::Mi355x`, its `parse` names, `validate`,
//! `create_attention_backend`, two `BackendPlan` variants and the `forward_into` arm).

use std::{
    cell::RefCell,
    collections::HashMap,
    ffi::c_void,
    rc::{Rc, Weak},
};

use mi355x_sys as sys;
use tch::{Device, Kind, Tensor};

use crate::engine::{
    AttentionMetadata, BatchPhase, DecodeGraphState, DecodeHostMetadata, MetadataRequirements,
};

use super::{
    AttentionBackend, AttentionSpec, BackendPlan, BaseAttention, FlashAttentionBackend,
    PrefillMetadata, Result, model_error,
};

/// An opaque native plan and the entry that frees it.
pub(super) struct Mi355xPlan {
    handle: *mut c_void,
    prefill: bool,
    /// The KV cache page size the plan was made for (the run entries check it).
    page_size: i64,
}

impl Drop for Mi355xPlan {
    fn drop(&mut self) {
        // The library waits for the plan's pending uploads before freeing it.
        unsafe {
            if self.prefill {
                sys::mi355x_prefill_plan_drop(self.handle)
            } else {
                sys::mi355x_decode_plan_drop(self.handle)
            }
        }
    }
}

#[derive(Default)]
pub(super) struct Mi355xAttentionBackend {
    plan: RefCell<Option<Rc<Mi355xPlan>>>,
    prefill_plan: RefCell<Option<Rc<Mi355xPlan>>>,
    graph_plans: RefCell<HashMap<usize, Weak<Mi355xPlan>>>,
}

fn dtype_code(kind: Kind) -> Result<i64> {
    match kind {
        Kind::BFloat16 => Ok(0),
        Kind::Half => Ok(1),
        _ => Err(model_error("mi355x attention requires bfloat16 or float16")),
    }
}

fn stream_of(device: Device) -> *mut c_void {
    match device {
        Device::Cuda(index) => sys::current_stream(index as i64),
        _ => std::ptr::null_mut(),
    }
}

fn check(status: *const std::ffi::c_char, what: &str) -> Result<()> {
    sys::check(status).map_err(|error| model_error(&format!("{what}: {error}")))
}

impl AttentionBackend for Mi355xAttentionBackend {
    fn metadata_requirements(&self, _phase: BatchPhase) -> MetadataRequirements {
        MetadataRequirements {
            block_table: true,
            req_to_token: false,
        }
    }

    fn supports_cuda_graph(&self) -> bool {
        true
    }

    fn prepare_decode_graph(
        &self,
        metadata: &AttentionMetadata,
        spec: AttentionSpec,
        page_size: i64,
    ) -> Result<Option<Box<dyn DecodeGraphState>>> {
        let table = metadata
            .block_table
            .as_ref()
            .ok_or_else(|| model_error("missing graph block_table"))?;
        let lengths = metadata
            .cache_seqlens
            .as_ref()
            .ok_or_else(|| model_error("missing graph cache_seqlens"))?;
        let plan = Rc::new(Mi355xPlan {
            handle: prepare_decode(metadata, spec, page_size, std::ptr::null_mut(), true)?,
            prefill: false,
            page_size,
        });
        let mut plans = self.graph_plans.borrow_mut();
        plans.retain(|_, plan| plan.strong_count() > 0);
        let key = table.data_ptr() as usize;
        if plans.get(&key).and_then(Weak::upgrade).is_some() {
            return Err(model_error("decode graph buffers are already registered"));
        }
        plans.insert(key, Rc::downgrade(&plan));
        Ok(Some(Box::new(Mi355xGraphState {
            plan,
            table: table.shallow_clone(),
            lengths: lengths.shallow_clone(),
            spec,
            page_size,
        })))
    }

    fn prepare(
        &self,
        metadata: Option<&AttentionMetadata>,
        prefill: &PrefillMetadata,
        spec: AttentionSpec,
        page_size: Option<i64>,
    ) -> Result<BackendPlan> {
        if let Some(metadata) = metadata.filter(|meta| meta.forward_mode == BatchPhase::Decode) {
            if let Some(plan) = metadata.block_table.as_ref().and_then(|table| {
                self.graph_plans
                    .borrow()
                    .get(&(table.data_ptr() as usize))
                    .and_then(Weak::upgrade)
            }) {
                // Planned outside capture/replay: no device read-back, no allocation.
                return Ok(BackendPlan::Mi355xDecode(plan));
            }
            let page_size =
                page_size.ok_or_else(|| model_error("mi355x requires a bound KV cache"))?;
            let mut cached = self.plan.borrow_mut();
            if cached
                .as_ref()
                .is_some_and(|plan| Rc::strong_count(plan) != 1)
            {
                return Err(model_error("previous mi355x batch is still in use"));
            }
            let existing = cached.as_ref().map_or(std::ptr::null_mut(), |plan| plan.handle);
            let handle = prepare_decode(metadata, spec, page_size, existing, false)?;
            let plan = cached.get_or_insert_with(|| {
                Rc::new(Mi355xPlan {
                    handle,
                    prefill: false,
                    page_size,
                })
            });
            return Ok(BackendPlan::Mi355xDecode(Rc::clone(plan)));
        }
        if let Some(metadata) = metadata {
            let mut cached = self.prefill_plan.borrow_mut();
            if cached
                .as_ref()
                .is_some_and(|plan| Rc::strong_count(plan) != 1)
            {
                return Err(model_error("previous mi355x prefill batch is still in use"));
            }
            let existing = cached.as_ref().map_or(std::ptr::null_mut(), |plan| plan.handle);
            let page_size =
                page_size.ok_or_else(|| model_error("mi355x requires a bound KV cache"))?;
            let handle = prepare_prefill(metadata, prefill, spec, page_size, existing)?;
            let plan = cached.get_or_insert_with(|| {
                Rc::new(Mi355xPlan {
                    handle,
                    prefill: true,
                    page_size,
                })
            });
            return Ok(BackendPlan::Mi355xPrefill(
                Rc::clone(plan),
                prefill.has_prefix(),
            ));
        }
        FlashAttentionBackend.prepare(metadata, prefill, spec, page_size)
    }

    fn forward(
        &self,
        q: &Tensor,
        k: &Tensor,
        v: &Tensor,
        cache: &BaseAttention,
        prefill: &PrefillMetadata,
        metadata: Option<&AttentionMetadata>,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        plan: &BackendPlan,
    ) -> Result<Tensor> {
        if metadata.is_some_and(|meta| meta.forward_mode == BatchPhase::Decode) {
            return mi355x_decode(q, cache, plan, num_kv_heads, head_dim, None);
        }
        if metadata.is_some() {
            return mi355x_prefill(q, k, v, cache, plan, num_kv_heads, head_dim, None);
        }
        FlashAttentionBackend.forward(
            q,
            k,
            v,
            cache,
            prefill,
            metadata,
            num_heads,
            num_kv_heads,
            head_dim,
            plan,
        )
    }
}

/// Graph-mode decode plan: fixed rows and columns, re-planned at a fixed address before
/// every replay (`FlashInferGraphState`, `backend.rs:490-530`).
struct Mi355xGraphState {
    plan: Rc<Mi355xPlan>,
    table: Tensor,
    lengths: Tensor,
    spec: AttentionSpec,
    page_size: i64,
}

impl DecodeGraphState for Mi355xGraphState {
    fn prepare_replay(&self, host: Option<&DecodeHostMetadata>) -> Result<()> {
        // Pad rows of the captured bucket read page 0 with length 1 and write slot 0.
        let host = host.map(|host| {
            let mut cache_seqlens = host.cache_seqlens.clone();
            cache_seqlens.resize(self.table.size()[0] as usize, 1);
            DecodeHostMetadata {
                cache_seqlens,
                block_table_versions: None,
            }
        });
        let metadata = AttentionMetadata {
            forward_mode: BatchPhase::Decode,
            decode_host: host,
            write_loc: None,
            cu_seqlens_q: None,
            prefix_lens: None,
            block_table: Some(self.table.shallow_clone()),
            cache_seqlens: Some(self.lengths.shallow_clone()),
            req_to_token: None,
            max_seqlen: None,
        };
        let handle = prepare_decode(&metadata, self.spec, self.page_size, self.plan.handle, true)?;
        if handle != self.plan.handle {
            return Err(model_error("graph plan address changed"));
        }
        Ok(())
    }

    fn needs_req_to_token(&self) -> bool {
        false
    }
}

/// `mi355x_decode_prepare` on the step's block table and lengths (the scheduler's host
/// lengths when present, so planning never reads the device back).
fn prepare_decode(
    metadata: &AttentionMetadata,
    spec: AttentionSpec,
    page_size: i64,
    existing: *mut c_void,
    graph: bool,
) -> Result<*mut c_void> {
    let table = metadata
        .block_table
        .as_ref()
        .ok_or_else(|| model_error("mi355x decode requires block_table"))?;
    let lengths = metadata
        .cache_seqlens
        .as_ref()
        .ok_or_else(|| model_error("mi355x decode requires cache_seqlens"))?;
    if table.dim() != 2 || table.kind() != Kind::Int || lengths.kind() != Kind::Int {
        return Err(model_error("invalid decode block table or lengths"));
    }
    let (rows, cols) = (table.size()[0], table.size()[1]);
    let host = metadata.decode_host.as_ref();
    let prepared = unsafe {
        sys::mi355x_decode_prepare(
            existing,
            table.data_ptr().cast(),
            rows,
            cols,
            table.stride()[0],
            lengths.data_ptr().cast(),
            spec.num_heads,
            spec.num_kv_heads,
            spec.head_dim,
            page_size,
            dtype_code(spec.kind)?,
            graph,
            host.map_or(std::ptr::null(), |host| host.cache_seqlens.as_ptr()),
            host.map_or(0, |host| host.cache_seqlens.len() as i64),
            stream_of(spec.device),
        )
    };
    if prepared.is_null() {
        return Err(model_error(&format!(
            "mi355x decode plan failed: {}",
            sys::last_error()
        )));
    }
    Ok(prepared)
}

/// `mi355x_prefill_prepare` from the host snapshot `Attention::prepare` already took
/// (`PrefillMetadata`), so the plan needs no device read-back.
fn prepare_prefill(
    metadata: &AttentionMetadata,
    prefill: &PrefillMetadata,
    spec: AttentionSpec,
    page_size: i64,
    existing: *mut c_void,
) -> Result<*mut c_void> {
    let cumulative = metadata
        .cu_seqlens_q
        .as_ref()
        .ok_or_else(|| model_error("missing cu_seqlens_q"))?;
    let table = metadata.block_table.as_ref();
    if prefill.has_prefix() && table.is_none() {
        return Err(model_error("missing block_table"));
    }
    let boundaries: Vec<i32> = prefill.boundaries.iter().map(|&v| v as i32).collect();
    let prefixes: Vec<i32> = prefill.prefixes.iter().map(|&v| v as i32).collect();
    let batch = prefixes.len() as i64;
    let prepared = unsafe {
        sys::mi355x_prefill_prepare(
            existing,
            cumulative.data_ptr().cast(),
            table.map_or(std::ptr::null(), |t| t.data_ptr().cast()),
            batch,
            table.map_or(0, |t| t.size()[1]),
            table.map_or(0, |t| t.stride()[0]),
            boundaries.as_ptr(),
            prefixes.as_ptr(),
            spec.num_heads,
            spec.num_kv_heads,
            page_size,
            dtype_code(spec.kind)?,
            stream_of(spec.device),
        )
    };
    if prepared.is_null() {
        return Err(model_error(&format!(
            "mi355x prefill plan failed: {}",
            sys::last_error()
        )));
    }
    Ok(prepared)
}

/// Paged decode into `output` ([tokens, heads * 128], contiguous) or a new tensor. The
/// query may be a strided view of packed QKV (no contiguous copy, unlike
/// `backend.rs:651`).
pub(super) fn mi355x_decode(
    q: &Tensor,
    cache: &BaseAttention,
    plan: &BackendPlan,
    num_kv_heads: i64,
    head_dim: i64,
    output: Option<&Tensor>,
) -> Result<Tensor> {
    if !matches!(q.device(), Device::Cuda(_)) {
        return Err(model_error("mi355x decode requires a GPU device"));
    }
    let BackendPlan::Mi355xDecode(plan) = plan else {
        return Err(model_error("mi355x decode requires a prepared batch"));
    };
    let (k_cache, v_cache) = cache.cache_tensors()?;
    let (tokens, heads) = (q.size()[0], q.size()[1]);
    let out = output.map_or_else(
        || Tensor::empty([tokens, heads * head_dim], (q.kind(), q.device())),
        Tensor::shallow_clone,
    );
    let qs = q.stride();
    check(
        unsafe {
            sys::mi355x_decode_run(
                plan.handle,
                q.data_ptr().cast_const(),
                qs[0],
                qs[1],
                k_cache.data_ptr().cast_const(),
                v_cache.data_ptr().cast_const(),
                out.data_ptr(),
                heads * head_dim,
                head_dim,
                tokens,
                heads,
                num_kv_heads,
                plan.page_size,
                dtype_code(q.kind())?,
                stream_of(q.device()),
            )
        },
        "mi355x decode failed",
    )?;
    Ok(out)
}

/// Ragged (no prefix) or paged (cached prefix) causal prefill, chosen once at prepare.
pub(super) fn mi355x_prefill(
    q: &Tensor,
    k: &Tensor,
    v: &Tensor,
    cache: &BaseAttention,
    plan: &BackendPlan,
    num_kv_heads: i64,
    head_dim: i64,
    output: Option<&Tensor>,
) -> Result<Tensor> {
    let BackendPlan::Mi355xPrefill(plan, paged) = plan else {
        return Err(model_error("missing mi355x prefill plan"));
    };
    // Paged plans read the layer's whole cache [pages, page, kv_heads, 128]; ragged plans
    // read the (packed) K/V projection rows in place.
    let cached;
    let (k, v, k_sn, k_sh, v_sn, v_sh) = if *paged {
        cached = cache.cache_tensors()?;
        let (kc, vc) = cached;
        let row = num_kv_heads * head_dim;
        (kc, vc, row, head_dim, row, head_dim)
    } else {
        let (ks, vs) = (k.stride(), v.stride());
        (k, v, ks[0], ks[1], vs[0], vs[1])
    };
    let (tokens, heads) = (q.size()[0], q.size()[1]);
    let out = output.map_or_else(
        || Tensor::empty([tokens, heads * head_dim], (q.kind(), q.device())),
        Tensor::shallow_clone,
    );
    let qs = q.stride();
    check(
        unsafe {
            sys::mi355x_prefill_run(
                plan.handle,
                q.data_ptr().cast_const(),
                qs[0],
                qs[1],
                k.data_ptr().cast_const(),
                k_sn,
                k_sh,
                v.data_ptr().cast_const(),
                v_sn,
                v_sh,
                out.data_ptr(),
                heads * head_dim,
                head_dim,
                tokens,
                heads,
                num_kv_heads,
                plan.page_size,
                dtype_code(q.kind())?,
                stream_of(q.device()),
            )
        },
        "mi355x prefill failed",
    )?;
    Ok(out)
}
