#pragma once

// Visibility of the public API of libsca_host.so. Only headers under include/scicompute_attention
// (plus the sci:: infrastructure headers) form the contract; everything else is internal.
//
// Conventions of the whole API:
//   * no exception crosses it: failures are sci::Status values (or sci::Result<T> for calls that
//     produce a value) whose message starts with "[SCA-<code>]";
//   * `stream == nullptr` means sci::Stream::GetCurrent().

#if defined(__GNUC__) || defined(__clang__)
#define SCI_ATTENTION_API __attribute__((visibility("default")))
#define SCI_ATTENTION_INTERNAL __attribute__((visibility("hidden")))
#else
#define SCI_ATTENTION_API
#define SCI_ATTENTION_INTERNAL
#endif
